// qnn_context.hip -- the resident context behind the C ABI (include/qnn_hip.h).
//
// Host-side counterpart of TQNNGPUContext
// (src/backends/vulkan/QuickNN.Vulkan.Context.Implementation.inc) and the
// weight cache of TQNNVulkan (src/backends/vulkan/QuickNN.Vulkan.pas:551-740),
// built on one HIP stream per context.
#include <algorithm>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "qnn_internal.h"

namespace qnn {

thread_local std::string t_last_error;
void set_last_error(const std::string &msg) { t_last_error = msg; }

struct GraphRec {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<WeightEntry *> pinned;
};

struct ExpertSetImpl;

}  // namespace qnn

struct qnn_tensor_s : qnn::Tensor {};

struct qnn_expert_set_s {
  int experts = 0, hidden = 0, inter = 0;
  qnn::I4Layout gu, dn;
  void *mem = nullptr;  // device: [gate x experts][up x experts][down x experts], tiled INT4
  size_t bytes = 0, source_bytes = 0;
};


struct qnn_ctx_s {
  int device = 0;
  hipStream_t stream = nullptr;
  std::thread::id owner;
  std::vector<qnn_tensor_s *> tensors;
  qnn_tensor_s *scratch[4] = {nullptr, nullptr, nullptr, nullptr};
  std::unordered_map<std::string, qnn::WeightEntry *> weights;
  uint64_t weight_bytes = 0, weight_limit = 0, clock = 0;
  int *error_flag = nullptr;
  // split-K workspace: partial sums + per-tile tickets (zeroed once, self-resetting)
  float *partial = nullptr;
  size_t partial_floats = 0;
  unsigned *counters = nullptr;
  size_t counter_count = 0;
  // generic workspace (MoE plan and hidden states, activation quantisation)
  void *work = nullptr;
  size_t work_bytes = 0;
  // upload staging
  void *staging = nullptr;
  size_t staging_bytes = 0;
  // pinned host readback buffer (data + error word)
  void *readback = nullptr;
  size_t readback_bytes = 0;
  // PreloadWeights pins until the next Flush/Download (Context.Implementation.inc:399-419);
  // RetainWeight pins for the context's lifetime (:361-387).
  std::vector<qnn::WeightEntry *> flush_pins;
  std::vector<qnn::WeightEntry *> retained;
  uint64_t retained_bytes = 0;
  // An INT4 TrySwiGLUVector recorded but not launched yet: the next call
  // either fuses it with the Int4Linear that reads its output (one launch for
  // the MLP, qnn_mlp.hip) or launches it on its own first.
  struct Pending {
    bool on = false;
    qnn::WeightEntry *g = nullptr, *u = nullptr;
    const float *x = nullptr;
    float *h = nullptr;
    int in = 0, out = 0;
  } pending;
  // Completion flags of the single-launch kernels (fused MLP, one-token MoE):
  // zeroed when allocated, then only ever set to launch epochs, which are
  // unique per context, so both share it.
  void *mlp_flags = nullptr;
  size_t mlp_flag_bytes = 0;
  unsigned mlp_epoch = 0;
  int mlp_cap[9][9] = {};
  int moe_cap[9][17] = {};  // co-resident workgroups of the one-token MoE kernel per (steps, route) variant
  // A one-token GO_MOE_ROUTE recorded instead of launched: when the next call
  // is qnn_moe_experts on its output, that launch computes the routes itself.
  struct PendingRoute {
    bool on = false;
    const float *logits = nullptr;
    float *routes = nullptr;
    int experts = 0, k = 0, normalize = 0;
  } proute;
  // GGUF one-row Linear calls recorded for one grouped launch: consecutive
  // calls on the same input (a layer's q/k/v or gate/up projections) with the
  // same encoding and plan width, at most kGGMaxGroup, distinct outputs.
  struct LinearGroup {
    int count = 0, bw = 0, enc = 0, enc2 = -1;  // enc2: a second K-quant encoding (one unit per wave), or -1
    const float *x = nullptr;
    qnn::WeightEntry *e[qnn::kGGMaxGroup] = {};
    float *y[qnn::kGGMaxGroup] = {};
    int out[qnn::kGGMaxGroup] = {}, slices[qnn::kGGMaxGroup] = {};
  } lgroup;  // co-resident workgroups of the fused MLP kernel per (gate/up, down) steps (0: not asked yet, -1: none)
  // Multi-row Int4Linear calls recorded to meet a GO_SWIGLU: the first, then
  // a second on the same input and shape; when the next call is GO_SWIGLU of
  // their two outputs, the three run as one gate/up SwiGLU launch.
  struct PendingRows {
    int count = 0;
    qnn::WeightEntry *e[2] = {};
    float *y[2] = {};
    const float *x = nullptr;
    int rows = 0, in = 0, out = 0;
  } prows;
  hipEvent_t events[64] = {};
  bool capturing = false;
  std::vector<qnn::WeightEntry *> capture_pins;
  std::vector<qnn::GraphRec> graphs;
  std::vector<qnn_expert_set_s *> sets;
  qnn_status st{};
  uint64_t act_bytes = 0;
  // OnWeightEvicted (Context.API.inc:164): told the identity of every entry
  // the cache evicts, before its memory is released (QuickNN.Vulkan.pas:568-569).
  qnn_weight_evicted_fn on_evicted = nullptr;
  void *on_evicted_user = nullptr;
  // Asynchronous layer prefetch (Context.Prefetch.inc): two slots, each with a
  // pinned host staging buffer, a raw device staging buffer and an event that
  // the copy stream records after the slot's copies and repacks.
  struct PrefetchSlot {
    void *host = nullptr;
    void *dev = nullptr;
    hipEvent_t ready = nullptr;
    bool submitted = false;
    std::vector<std::string> keys;
    std::vector<qnn::WeightEntry *> entries;  // one pin each while queued or active
    std::vector<std::string> prepared_keys;   // host staging filled by StageWeightPrefetch
    std::vector<uint64_t> prepared_offsets;
  };
  struct Prefetch {
    bool enabled = false;
    uint64_t bytes = 0;
    hipStream_t copy = nullptr;
    PrefetchSlot slot[2];
    int active = -1, queued = -1, next = 0;
  } pf;
};

namespace qnn {
namespace {
Tuning g_tuning;
int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}
}  // namespace

const Tuning &tuning() { return g_tuning; }
void reload_tuning() {
  Tuning t;
  t.group_linear = env_int("QNN_GROUP_LINEAR", t.group_linear);
  t.fuse_mlp = env_int("QNN_FUSE_MLP", t.fuse_mlp);
  t.fuse_moe = env_int("QNN_FUSE_MOE", t.fuse_moe);
  t.q8_gemm_min_rows = env_int("QNN_Q8_GEMM_MIN_ROWS", t.q8_gemm_min_rows);
  t.gemm_h16 = env_int("QNN_GEMM_H16", t.gemm_h16);
  t.gguf_gemm_rows = env_int("QNN_GGUF_GEMM_ROWS", t.gguf_gemm_rows);
  t.gemm_max_rows = env_int("QNN_GEMM_MAX_ROWS", t.gemm_max_rows);
  t.attn_wgs = env_int("QNN_ATTN_WGS", t.attn_wgs);
  t.attn_min_chunk = env_int("QNN_ATTN_MIN_CHUNK", t.attn_min_chunk);
  t.attn_dma = env_int("QNN_ATTN_DMA", t.attn_dma);
  t.gemm_nw = env_int("QNN_GEMM_NW", t.gemm_nw);
  t.gemm_mb = env_int("QNN_GEMM_MB", t.gemm_mb);
  t.gg_bw = env_int("QNN_GG_BW", t.gg_bw);
  t.gg_mt = env_int("QNN_GG_MT", t.gg_mt);
  t.i4_mfma = env_int("QNN_I4_MFMA", t.i4_mfma);
  t.i4_lanes = env_int("QNN_I4_LANES", t.i4_lanes);
  t.i4_tpw = env_int("QNN_I4_TPW", t.i4_tpw);
  t.i4_target_waves = env_int("QNN_I4_TARGET_WAVES", t.i4_target_waves);
  t.i4_sps = env_int("QNN_I4_SPS", t.i4_sps);
  t.i4_wide = env_int("QNN_I4_WIDE", t.i4_wide);
  t.moe_mt = env_int("QNN_MOE_MT", t.moe_mt);
  t.moe_sps = env_int("QNN_MOE_SPS", t.moe_sps);
  g_tuning = t;
}

namespace {

std::mutex g_lock;
qnn_ctx_s *g_ctx = nullptr;

template <typename F>
int guarded(F &&f) {
  try {
    return f();
  } catch (const Error &e) {
    t_last_error = e.what();
    return e.code;
  } catch (const std::bad_alloc &) {
    t_last_error = "host allocation failed";
    return QNN_E_RANGE;
  } catch (const std::exception &e) {
    t_last_error = e.what();
    return QNN_E_INVALID_OP;
  }
}

void settle_pending(qnn_ctx_s *ctx);
void run_gguf(qnn_ctx_s *ctx, const WeightEntry *w, const WeightEntry *w2, int mode, const float *x, float *y,
              int out_dim, float *g_out = nullptr, float *u_out = nullptr);

// Every entry point starts here.  A recorded SwiGLU is launched first unless
// the caller is the Int4Linear that may fuse with it (keep_pending).
void check_ctx(qnn_ctx_s *ctx, bool keep_pending = false) {
  if (!ctx || ctx != g_ctx) fail(QNN_E_ARGUMENT, "invalid context");
  // Context.Implementation.inc:70-71: resident work stays on its creating thread.
  if (std::this_thread::get_id() != ctx->owner) fail(QNN_E_INVALID_OP, "context used from a thread other than its creator");
  hip_check(hipSetDevice(ctx->device), "hipSetDevice");
  if (!keep_pending && (ctx->pending.on || ctx->lgroup.count || ctx->proute.on || ctx->prows.count)) settle_pending(ctx);
}

// Check (Context.Implementation.inc): a live tensor of at least `minimum` floats.
void check_tensor(qnn_ctx_s *ctx, const qnn_tensor_s *t, int64_t minimum = 1) {
  if (!t) fail(QNN_E_ARGUMENT, "missing tensor");
  bool owned = std::find(ctx->tensors.begin(), ctx->tensors.end(), t) != ctx->tensors.end();
  if (!owned || !t->live) fail(QNN_E_ARGUMENT, "tensor is not live in this context");
  if (int64_t(t->count) < minimum) fail(QNN_E_ARGUMENT, "tensor too small for the operation");
}

void sync(qnn_ctx_s *ctx) {
  if (ctx->capturing) fail(QNN_E_INVALID_OP, "synchronisation requested during graph capture");
  hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  ctx->st.submissions++;
}


// Flush releases the pins a synchronous preload took (Context.Implementation.inc:411-415).
void release_flush_pins(qnn_ctx_s *ctx) {
  for (auto *e : ctx->flush_pins) e->pins--;
  ctx->flush_pins.clear();
}

// ---------------------------------------------------------------- tensors
qnn_tensor_s *new_tensor(qnn_ctx_s *ctx, int count) {
  if (count < 1) fail(QNN_E_RANGE, "resident tensor size");
  const size_t bytes = size_t(count) * 4;
  qnn_tensor_s *best = nullptr;
  for (auto *t : ctx->tensors)  // best-fit reuse (Context.Implementation.inc:123-127)
    if (!t->live && t->capacity >= bytes && (!best || t->capacity < best->capacity)) best = t;
  if (!best) {
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "tensor allocation during graph capture");
    best = new qnn_tensor_s();
    const size_t cap = (bytes + 255) & ~size_t(255);
    if (hipMalloc(&best->ptr, cap) != hipSuccess) {
      delete best;
      (void)hipGetLastError();
      fail(QNN_E_RANGE, "GPU activation allocation failed");
    }
    best->capacity = cap;
    ctx->tensors.push_back(best);
    ctx->act_bytes += cap;
    ctx->st.activation_bytes = ctx->act_bytes;
    ctx->st.activation_peak_bytes = std::max(ctx->st.activation_peak_bytes, ctx->act_bytes);
  }
  best->count = count;
  best->live = true;
  return best;
}

// ---------------------------------------------------------------- workspace
void ensure_splitk(qnn_ctx_s *ctx, size_t partial_floats, size_t counters) {
  if (partial_floats <= ctx->partial_floats && counters <= ctx->counter_count) return;
  if (ctx->capturing) fail(QNN_E_INVALID_OP, "split-K workspace growth during graph capture (run the sequence once first)");
  sync(ctx);
  partial_floats = std::max(partial_floats, ctx->partial_floats);
  counters = std::max(counters, ctx->counter_count);
  if (ctx->partial) (void)hipFree(ctx->partial);
  if (ctx->counters) (void)hipFree(ctx->counters);
  ctx->partial = nullptr;
  ctx->counters = nullptr;
  hip_check(hipMalloc(&ctx->partial, std::max<size_t>(partial_floats, 1) * 4), "workspace allocation");
  hip_check(hipMalloc(&ctx->counters, std::max<size_t>(counters, 1) * 4), "workspace allocation");
  // On the context stream and waited for: a plain hipMemset runs on the null
  // stream, which a non-blocking stream does not wait for, so the next kernel
  // could read tickets left in the recycled allocation.
  hip_check(hipMemsetAsync(ctx->counters, 0, std::max<size_t>(counters, 1) * 4, ctx->stream), "workspace clear");
  hip_check(hipStreamSynchronize(ctx->stream), "workspace clear");
  ctx->partial_floats = partial_floats;
  ctx->counter_count = counters;
}

void *ensure_work(qnn_ctx_s *ctx, size_t bytes) {
  if (bytes <= ctx->work_bytes) return ctx->work;
  if (ctx->capturing) fail(QNN_E_INVALID_OP, "workspace growth during graph capture (run the sequence once first)");
  sync(ctx);
  if (ctx->work) (void)hipFree(ctx->work);
  ctx->work = nullptr;
  hip_check(hipMalloc(&ctx->work, bytes), "workspace allocation");
  ctx->work_bytes = bytes;
  return ctx->work;
}

void *ensure_staging(qnn_ctx_s *ctx, size_t bytes) {
  if (bytes <= ctx->staging_bytes) return ctx->staging;
  if (ctx->staging) (void)hipFree(ctx->staging);
  ctx->staging = nullptr;
  ctx->staging_bytes = 0;
  if (hipMalloc(&ctx->staging, bytes) != hipSuccess) {
    (void)hipGetLastError();
    fail(QNN_E_RANGE, "weight upload staging allocation failed");
  }
  ctx->staging_bytes = bytes;
  return ctx->staging;
}

// ---------------------------------------------------------------- weight cache
int gguf_block_elements(int enc) {  // GGUF.Quantization.pas:67-75 (formats in this backend)
  switch (enc) {
    case QNN_WE_Q8_0: case QNN_WE_IQ4_NL: return 32;
    case QNN_WE_Q2_0: return 64;
    case QNN_WE_IQ2_XXS: case QNN_WE_IQ2_S: case QNN_WE_IQ3_XXS: case QNN_WE_IQ3_S:
    case QNN_WE_Q4_K: case QNN_WE_Q6_K: case QNN_WE_Q3_K: case QNN_WE_Q2_K: case QNN_WE_Q5_K: case QNN_WE_IQ4_XS:
      return 256;
  }
  return -1;
}
int gguf_block_bytes(int enc) {  // GGUF.Quantization.pas:77-93
  switch (enc) {
    case QNN_WE_Q8_0: return 34;
    case QNN_WE_Q4_K: return 144;
    case QNN_WE_Q6_K: return 210;
    case QNN_WE_Q3_K: return 110;
    case QNN_WE_Q2_K: return 84;
    case QNN_WE_Q5_K: return 176;
    case QNN_WE_IQ4_NL: return 18;
    case QNN_WE_IQ4_XS: return 136;
    case QNN_WE_Q2_0: return 18;
    case QNN_WE_IQ2_XXS: return 66;
    case QNN_WE_IQ2_S: return 82;
    case QNN_WE_IQ3_XXS: return 98;
    case QNN_WE_IQ3_S: return 110;
  }
  return -1;
}
bool is_gguf(int enc) { return enc != QNN_WE_NATIVE; }

void check_weight_desc(const qnn_weight *w) {
  if (!w) fail(QNN_E_ARGUMENT, "missing weight");
  if (w->identity == 0 || !w->data) fail(QNN_E_ARGUMENT, "Weight must have immutable identity and assigned storage");
}

// GGUFWeightBytes (GGUF.Quantization.pas:105-113).
uint64_t gguf_weight_bytes(const qnn_weight *w, int rows, int cols) {
  const int be = gguf_block_elements(w->encoding);
  if (be < 0) fail(QNN_E_NOT_SUPPORTED, "GGUF encoding not supported by the HIP backend");
  if (w->dtype != QNN_DT_U8 || rows < 1 || cols < 1 || cols % be != 0 || w->offset < 0 || w->offset % be != 0 ||
      int64_t(rows) * cols > w->size - w->offset)
    fail(QNN_E_ARGUMENT, "Invalid packed GGUF matrix span");
  return uint64_t(int64_t(rows) * cols / be) * uint64_t(gguf_block_bytes(w->encoding));
}

// WeightKey (QuickNN.Vulkan.pas:641-662): identity/dtype:encoding/offset/bytes.
std::string weight_key(const char *kind, const qnn_weight *w, uint64_t bytes) {
  char buf[160];
  snprintf(buf, sizeof buf, "%s/%016" PRIx64 "/%d:%d/%" PRId64 "/%" PRIu64, kind, w->identity, w->dtype, w->encoding,
           w->offset, bytes);
  return buf;
}

void evict_one_or_fail(qnn_ctx_s *ctx) {  // EvictOne (QuickNN.Vulkan.pas:551-579): LRU of unpinned entries
  qnn::WeightEntry *oldest = nullptr;
  for (auto &kv : ctx->weights) {
    auto *e = kv.second;
    if (e->pins == 0 && e->op_pins == 0 && (!oldest || e->last_use < oldest->last_use)) oldest = e;
  }
  if (!oldest) fail(QNN_E_RANGE, "VRAM cache cannot hold the active chain");
  if (ctx->on_evicted && !oldest->derived) ctx->on_evicted(oldest->identity, ctx->on_evicted_user);
  ctx->weights.erase(oldest->key);
  ctx->weight_bytes -= oldest->bytes;
  (void)hipFree(oldest->dptr);
  delete oldest;
  ctx->st.weight_evictions++;
}

void make_room(qnn_ctx_s *ctx, size_t bytes) {
  if (bytes > ctx->weight_limit) fail(QNN_E_RANGE, "Weight exceeds VRAM cache limit");
  while (ctx->weight_bytes + bytes > ctx->weight_limit) evict_one_or_fail(ctx);
}

WeightEntry *lookup(qnn_ctx_s *ctx, const std::string &key) {
  auto it = ctx->weights.find(key);
  if (it == ctx->weights.end()) return nullptr;
  it->second->last_use = ++ctx->clock;
  ctx->st.weight_cache_hits++;
  if (it->second->ready) {  // written by a prefetch: compute waits for its copy stream first
    if (ctx->capturing) hip_check(hipEventSynchronize(it->second->ready), "prefetch join");
    else hip_check(hipStreamWaitEvent(ctx->stream, it->second->ready, 0), "prefetch join");
    it->second->ready = nullptr;
  }
  if (ctx->capturing) {
    it->second->pins++;
    ctx->capture_pins.push_back(it->second);
  }
  return it->second;
}

WeightEntry *insert(qnn_ctx_s *ctx, WeightEntry *e) {
  e->last_use = ++ctx->clock;
  ctx->weights[e->key] = e;
  ctx->weight_bytes += e->bytes;
  if (!e->derived) {  // a copy made on the device is not an upload
    ctx->st.weight_uploads++;
    ctx->st.weight_upload_bytes += e->source_bytes;
  }
  return e;
}

void begin_miss(qnn_ctx_s *ctx) {
  ctx->st.weight_cache_misses++;
  if (ctx->capturing) fail(QNN_E_INVALID_OP, "weight not resident during graph capture (preload it first)");
  sync(ctx);  // AcquireWeight flushes the resident context on a miss (QuickNN.Vulkan.pas:687-688)
}

void *alloc_weight(qnn_ctx_s *ctx, size_t bytes) {
  make_room(ctx, bytes);
  void *p = nullptr;
  while (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    evict_one_or_fail(ctx);  // device memory fragmented or shared: yield another unpinned entry
  }
  return p;
}

// Native INT4 matrix [rows, Int4RowBytes(cols)] -> tiled device copy.
WeightEntry *acquire_int4(qnn_ctx_s *ctx, const qnn_weight *w, int rows, int cols) {
  check_weight_desc(w);
  const int rb = qnn_int4_row_bytes(cols);
  if (w->dtype != QNN_DT_U8 || w->encoding != QNN_WE_NATIVE || w->offset != 0 || rb < 0 || w->shape0 != rows ||
      w->shape1 != rb || int64_t(rows) * rb > w->size)
    fail(QNN_E_ARGUMENT, "Invalid packed INT4 projection");
  const uint64_t bytes = uint64_t(rows) * rb;
  const std::string key = weight_key("i4", w, bytes);
  if (auto *e = lookup(ctx, key)) return e;
  begin_miss(ctx);
  auto *e = new WeightEntry();
  e->key = key;
  e->identity = w->identity;
  e->kind = WKind::Int4;
  e->i4 = int4_layout(rows, cols);
  e->bytes = e->i4.bytes();
  e->source_bytes = bytes;
  try {
    e->dptr = alloc_weight(ctx, e->bytes);
    void *stg = ensure_staging(ctx, bytes);
    hip_check(hipMemcpyAsync(stg, w->data, bytes, hipMemcpyHostToDevice, ctx->stream), "weight upload");
    int4_repack_launch(static_cast<const uint8_t *>(stg), e->i4, e->dptr, ctx->stream);
    sync(ctx);  // host storage need only stay valid during acquisition
  } catch (...) {
    if (e->dptr) (void)hipFree(e->dptr);
    delete e;
    throw;
  }
  return insert(ctx, e);
}

// GGUF matrix [rows, cols] elements -> tiled device copy.
WeightEntry *acquire_gguf(qnn_ctx_s *ctx, const qnn_weight *w, int rows, int cols) {
  check_weight_desc(w);
  const uint64_t bytes = gguf_weight_bytes(w, rows, cols);
  const std::string key = weight_key("gg", w, bytes);
  if (auto *e = lookup(ctx, key)) return e;
  begin_miss(ctx);
  auto *e = new WeightEntry();
  e->key = key;
  e->identity = w->identity;
  e->kind = WKind::Gguf;
  e->gg = gguf_layout(w->encoding, rows, cols);
  e->bytes = e->gg.bytes();
  e->source_bytes = bytes;
  try {
    e->dptr = alloc_weight(ctx, e->bytes);
    void *stg = ensure_staging(ctx, bytes);
    // GGUFWeightPointer (GGUF.Quantization.pas:115-121): the slice starts at
    // the quant bytes of `offset` elements.
    const uint8_t *src = static_cast<const uint8_t *>(w->data) +
                         uint64_t(w->offset / gguf_block_elements(w->encoding)) * gguf_block_bytes(w->encoding);
    hip_check(hipMemcpyAsync(stg, src, bytes, hipMemcpyHostToDevice, ctx->stream), "weight upload");
    gguf_repack_launch(static_cast<const uint8_t *>(stg), e->gg, e->dptr, ctx->stream);
    if (e->gg.rowexp_off) q8_rowexp_launch(e->gg, e->dptr, ctx->stream);
    sync(ctx);
  } catch (...) {
    if (e->dptr) (void)hipFree(e->dptr);
    delete e;
    throw;
  }
  return insert(ctx, e);
}

// F32/BF16 vector (norm gamma, bias) copied as is.
WeightEntry *acquire_raw(qnn_ctx_s *ctx, const qnn_weight *w, int64_t count, bool allow_s8 = false) {
  check_weight_desc(w);
  if ((w->dtype != QNN_DT_F32 && w->dtype != QNN_DT_BF16 && !(allow_s8 && w->dtype == QNN_DT_S8)) ||
      w->encoding != QNN_WE_NATIVE || w->offset < 0 || count > w->size - w->offset)
    fail(QNN_E_ARGUMENT, "vector weight must be F32 or BF16 with enough elements");
  const int es = w->dtype == QNN_DT_F32 ? 4 : w->dtype == QNN_DT_BF16 ? 2 : 1;
  const uint64_t bytes = uint64_t(count) * es;
  const std::string key = weight_key("raw", w, bytes);
  if (auto *e = lookup(ctx, key)) return e;
  begin_miss(ctx);
  auto *e = new WeightEntry();
  e->key = key;
  e->identity = w->identity;
  e->kind = WKind::Raw;
  e->raw_dtype = w->dtype;
  e->bytes = (bytes + 255) & ~uint64_t(255);
  e->source_bytes = bytes;
  try {
    e->dptr = alloc_weight(ctx, e->bytes);
    // Ordered on the context stream (a plain hipMemcpy from pageable memory may
    // return before its DMA lands, and the non-blocking stream would not wait).
    hip_check(hipMemcpyAsync(e->dptr, static_cast<const uint8_t *>(w->data) + w->offset * es, bytes,
                             hipMemcpyHostToDevice, ctx->stream),
              "vector upload");
    sync(ctx);
  } catch (...) {
    if (e->dptr) (void)hipFree(e->dptr);
    delete e;
    throw;
  }
  return insert(ctx, e);
}

// ---------------------------------------------------------------- asynchronous prefetch
// PrefetchWeights / StageWeightPrefetch accept complete 2-D matrices only
// (Context.Prefetch.inc:186-191, :328-333).
void check_prefetch_matrix(const qnn_weight *w) {
  check_weight_desc(w);
  if (w->offset != 0 || w->shape0 < 1 || w->shape0 > 0x7fffffff || w->shape1 < 1 || w->shape1 > 0x7fffffff ||
      w->size != w->shape0 * w->shape1)
    fail(QNN_E_ARGUMENT, "Layer prefetch requires complete immutable matrices");
}
// Source bytes of a matrix and the cache key its acquisition uses.
uint64_t matrix_source_bytes(const qnn_weight *w) {
  const int rows = int(w->shape0), cols = int(w->shape1);
  if (is_gguf(w->encoding)) return gguf_weight_bytes(w, rows, cols);
  if (w->dtype == QNN_DT_U8) return uint64_t(rows) * cols;
  if (w->dtype == QNN_DT_F32 || w->dtype == QNN_DT_BF16) return uint64_t(rows) * cols * (w->dtype == QNN_DT_F32 ? 4 : 2);
  fail(QNN_E_NOT_SUPPORTED, "only packed INT4, GGUF, F32 and BF16 matrices are resident in the HIP backend");
}
std::string matrix_key(const qnn_weight *w) {
  const uint64_t bytes = matrix_source_bytes(w);
  if (is_gguf(w->encoding)) return weight_key("gg", w, bytes);
  if (w->dtype == QNN_DT_U8) return weight_key("i4", w, bytes);
  return weight_key("raw", w, bytes);
}

// Waits for the slot's copies, unpins its entries and forgets its batch.
void release_slot(qnn_ctx_s *ctx, int i) {
  if (i < 0) return;
  qnn_ctx_s::PrefetchSlot &s = ctx->pf.slot[i];
  if (s.submitted) {
    hip_check(hipEventSynchronize(s.ready), "prefetch slot");
    s.submitted = false;
  }
  for (auto *e : s.entries) {
    if (e->ready == s.ready) e->ready = nullptr;  // complete; the event will be recorded again
    e->pins--;
  }
  s.entries.clear();
  s.keys.clear();
}

// A cache entry for matrix w, uploaded on the copy stream from the slot's
// staging at byte `off` (the host bytes are copied there first unless
// StageWeightPrefetch already did).
WeightEntry *prefetch_entry(qnn_ctx_s *ctx, qnn_ctx_s::PrefetchSlot &s, const qnn_weight *w, const std::string &key,
                            uint64_t bytes, uint64_t off, bool staged) {
  auto *e = new WeightEntry();
  e->key = key;
  e->identity = w->identity;
  e->source_bytes = bytes;
  const int rows = int(w->shape0), cols = int(w->shape1);
  if (is_gguf(w->encoding)) {
    e->kind = WKind::Gguf;
    e->gg = gguf_layout(w->encoding, rows, cols);
    e->bytes = e->gg.bytes();
  } else if (w->dtype == QNN_DT_U8) {
    const int k = (cols / 20) * 32;
    if (w->encoding != QNN_WE_NATIVE || qnn_int4_row_bytes(k) != cols) fail(QNN_E_ARGUMENT, "Invalid packed INT4 projection");
    e->kind = WKind::Int4;
    e->i4 = int4_layout(rows, k);
    e->bytes = e->i4.bytes();
  } else {
    e->kind = WKind::Raw;
    e->raw_dtype = w->dtype;
    e->bytes = (bytes + 255) & ~uint64_t(255);
  }
  try {
    e->dptr = alloc_weight(ctx, e->bytes);
    uint8_t *host = static_cast<uint8_t *>(s.host) + off;
    uint8_t *dev = static_cast<uint8_t *>(s.dev) + off;
    if (!staged) std::memcpy(host, w->data, bytes);
    hipStream_t cs = ctx->pf.copy;
    if (e->kind == WKind::Raw) {
      hip_check(hipMemcpyAsync(e->dptr, host, bytes, hipMemcpyHostToDevice, cs), "prefetch copy");
    } else {
      hip_check(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, cs), "prefetch copy");
      if (e->kind == WKind::Int4) {
        int4_repack_launch(dev, e->i4, e->dptr, cs);
      } else {
        gguf_repack_launch(dev, e->gg, e->dptr, cs);
        if (e->gg.rowexp_off) q8_rowexp_launch(e->gg, e->dptr, cs);
      }
    }
  } catch (...) {
    if (e->dptr) (void)hipFree(e->dptr);
    delete e;
    throw;
  }
  e->ready = s.ready;
  e->pins++;  // the slot's
  ctx->st.weight_cache_misses++;
  return insert(ctx, e);
}

void destroy_prefetch(qnn_ctx_s *ctx) {
  qnn_ctx_s::Prefetch &pf = ctx->pf;
  if (pf.copy) (void)hipStreamSynchronize(pf.copy);
  for (auto &s : pf.slot) {
    for (auto *e : s.entries) {
      if (e->ready == s.ready) e->ready = nullptr;
      e->pins--;
    }
    if (s.host) (void)hipHostFree(s.host);
    if (s.dev) (void)hipFree(s.dev);
    if (s.ready) (void)hipEventDestroy(s.ready);
    s = qnn_ctx_s::PrefetchSlot();
  }
  if (pf.copy) (void)hipStreamDestroy(pf.copy);
  pf = qnn_ctx_s::Prefetch();
}

// Holds entries against eviction for the duration of one call.
struct OpPins {
  std::vector<WeightEntry *> held;
  ~OpPins() {
    for (auto *e : held) e->op_pins--;
  }
  WeightEntry *operator()(WeightEntry *e) {
    e->op_pins++;
    held.push_back(e);
    return e;
  }
};

// ---------------------------------------------------------------- INT4 projection
// Caller-provided split-K workspace (the no-allocation entry point's static
// scratch): its tickets are cleared by a fill kernel before every launch.
struct FixedWs {
  float *partial = nullptr;
  unsigned *counters = nullptr;
};

void run_int4(qnn_ctx_s *ctx, const WeightEntry *w, const WeightEntry *w2, int mode, const float *x, float *y,
              int rows, int in_dim, int out_dim, const float *prob, float *g_out = nullptr, float *u_out = nullptr,
              const FixedWs *fixed = nullptr) {
  const I4Layout &l = w->i4;
  // The kernels read activation rows as aligned 4-float pieces: a row length
  // that is not a multiple of 4 goes through a zero-padded copy.
  int k = in_dim;
  qnn_tensor_s *padded = nullptr;
  if (in_dim % 4 != 0) {
    k = (in_dim + 3) / 4 * 4;
    padded = new_tensor(ctx, rows * k);
    misc_pad_rows(padded->ptr, x, rows, in_dim, k, ctx->stream);
    x = padded->ptr;
  }
  for (int r0 = 0; r0 < rows; r0 += 16) {
    const int m = std::min(16, rows - r0);
    I4Launch a;
    a.nib = w->dptr;
    a.scl = static_cast<const uint8_t *>(w->dptr) + l.nib_bytes();
    if (w2) {
      a.nib2 = w2->dptr;
      a.scl2 = static_cast<const uint8_t *>(w2->dptr) + l.nib_bytes();
    }
    a.x = x + size_t(r0) * k;
    a.x_stride = k;
    a.y = y + size_t(r0) * out_dim;
    a.y_stride = out_dim;
    a.k = k;
    a.n = out_dim;
    a.m = m;
    a.l = l;
    a.tiles = mode == I4_SWIGLU ? 2 * l.blocks : l.blocks;
    a.mode = mode;
    a.prob = prob;
    if (g_out) {
      a.g_out = g_out + size_t(r0) * out_dim;
      a.u_out = u_out + size_t(r0) * out_dim;
    }
    const I4Plan p = int4_plan(l, m, mode, true);
    if (fixed) {
      misc_fill(reinterpret_cast<float *>(fixed->counters), int(p.counters), 0u, ctx->stream);
      a.partial = fixed->partial;
      a.counters = fixed->counters;
    } else {
      ensure_splitk(ctx, p.partial_floats, p.counters);
      a.partial = ctx->partial;
      a.counters = ctx->counters;
    }
    a.err = ctx->error_flag;
    int4_matvec_launch(a, p, ctx->stream);
  }
  if (padded) padded->live = false;  // later users of the buffer are ordered after this launch
}

// ---------------------------------------------------------------- recorded ops
// Launches the recorded GGUF Linear group: one kernel, each member with its
// own split-K workspace, computed exactly as on its own.
void launch_linear_group(qnn_ctx_s *ctx) {
  qnn_ctx_s::LinearGroup g = ctx->lgroup;
  ctx->lgroup = {};
  for (int i = 0; i < g.count; ++i) g.e[i]->pins--;
  size_t pf = 0, nc = 0;
  GGGroup grp;
  grp.count = g.count;
  for (int i = 0; i < g.count; ++i) {
    const int tiles = g.e[i]->gg.tiles;
    grp.start[i + 1] = grp.start[i] + (tiles + 7) / 8 * 8 * g.slices[i];
    pf += g.slices[i] > 1 ? size_t(tiles) * g.slices[i] * 64 : 0;
    nc += size_t(tiles) * kCounterStride;
  }
  ensure_splitk(ctx, pf, nc);
  pf = nc = 0;
  for (int i = 0; i < g.count; ++i) {
    GGArgs &a = grp.m[i];
    const WeightEntry *w = g.e[i];
    a.l = w->gg;
    a.w = w->dptr;
    a.x = g.x;
    a.x_vec4 = (w->gg.cols % 4 == 0) && (reinterpret_cast<uintptr_t>(g.x) % 16 == 0);
    a.y = g.y[i];
    a.n = g.out[i];
    a.tiles = w->gg.tiles;
    a.mode = GG_STORE;
    a.partial = ctx->partial + pf;
    a.counters = ctx->counters + nc;
    a.err = ctx->error_flag;
    grp.slices[i] = g.slices[i];
    pf += g.slices[i] > 1 ? size_t(a.tiles) * g.slices[i] * 64 : 0;
    nc += size_t(a.tiles) * kCounterStride;
  }
  gguf_group_launch(grp, g.bw, ctx->stream);
  if (g.count > 1) ctx->st.linear_grouped += uint64_t(g.count);
}

bool linear_grouping_enabled() { return tuning().group_linear != 0; }

// A recorded one-row GGUF group of exactly a gate and an up projection of one
// shape, completed by a GLU of their two outputs: one gate/up pair launch
// (GG_SWIGLU / GG_GEGLU) that also writes both outputs.  Only where the pair
// launch's plan has the group's units per wave and slices, so every output
// is bit-identical to the grouped launch followed by the GLU.
bool try_glu_group(qnn_ctx_s *ctx, int op, int n, int interleaved, qnn_tensor_s *dst, qnn_tensor_s *a,
                   qnn_tensor_s *b) {
  const qnn_ctx_s::LinearGroup &g = ctx->lgroup;
  if (g.count != 2 || interleaved || !b || a->ptr != g.y[0] || b->ptr != g.y[1] || dst->ptr == g.x) return false;
  const GGLayout &l0 = g.e[0]->gg, &l1 = g.e[1]->gg;
  if (l0.enc != l1.enc || l0.rows != l1.rows || l0.cols != l1.cols || g.out[0] != g.out[1] || n != g.out[0])
    return false;
  int bw = 0, slices = 0;
  gguf_plan(l0, (g.out[0] + 31) / 32, &bw, &slices);
  if (bw != g.bw || slices != g.slices[0] || slices != g.slices[1]) return false;
  const qnn_ctx_s::LinearGroup q = g;
  ctx->lgroup = {};
  q.e[0]->pins--;
  q.e[1]->pins--;
  run_gguf(ctx, q.e[0], q.e[1], op == QNN_GO_GEGLU ? GG_GEGLU : GG_SWIGLU, q.x, dst->ptr, q.out[0], q.y[0], q.y[1]);
  ctx->st.glu_fused++;
  return true;
}

// Records a one-row GGUF Linear into the group, launching what was recorded
// first when it does not fit.
void record_linear(qnn_ctx_s *ctx, WeightEntry *e, const float *x, float *y, int out_dim) {
  int bw, slices;
  gguf_plan(e->gg, e->gg.tiles, &bw, &slices);
  qnn_ctx_s::LinearGroup &g = ctx->lgroup;
  // A second encoding may join (a layer's q/k/v often mix quant types): K-quants
  // at one unit per wave, at most two encodings per launch.
  const int enc = e->gg.enc;
  auto mixable = [](int v) {  // the K-quants k_gguf_matvec_mixed is built for
    return v == QNN_WE_Q4_K || v == QNN_WE_Q6_K || v == QNN_WE_Q3_K || v == QNN_WE_Q2_K;
  };
  const bool enc_ok = g.enc == enc || (bw == 1 && mixable(enc) && mixable(g.enc) && (g.enc2 < 0 || g.enc2 == enc));
  bool fits = g.count > 0 && g.count < kGGMaxGroup && g.x == x && enc_ok && g.bw == bw;
  for (int i = 0; fits && i < g.count; ++i) fits = g.y[i] != y;
  if (!fits) settle_pending(ctx);
  if (g.count == 0) {
    g.x = x;
    g.enc = enc;
    g.enc2 = -1;
    g.bw = bw;
  } else if (enc != g.enc) {
    g.enc2 = enc;
  }
  e->pins++;
  g.e[g.count] = e;
  g.y[g.count] = y;
  g.out[g.count] = out_dim;
  g.slices[g.count] = slices;
  g.count++;
  // The group's launch workspace, sized now so that launching it never allocates.
  size_t pf = 0, nc = 0;
  for (int i = 0; i < g.count; ++i) {
    pf += g.slices[i] > 1 ? size_t(g.e[i]->gg.tiles) * g.slices[i] * 64 : 0;
    nc += size_t(g.e[i]->gg.tiles) * kCounterStride;
  }
  ensure_splitk(ctx, pf, nc);
}

// ---------------------------------------------------------------- fused decode MLP
void settle_pending(qnn_ctx_s *ctx) {
  if (ctx->proute.on) {
    const qnn_ctx_s::PendingRoute r = ctx->proute;
    ctx->proute = {};
    misc_moe_route(r.routes, r.logits, 1, r.experts, r.k, r.normalize, ctx->stream);
  }
  if (ctx->lgroup.count) launch_linear_group(ctx);
  if (ctx->prows.count) {
    const qnn_ctx_s::PendingRows q = ctx->prows;
    ctx->prows = {};
    for (int i = 0; i < q.count; ++i) {
      q.e[i]->pins--;
      run_int4(ctx, q.e[i], nullptr, I4_STORE, q.x, q.y[i], q.rows, q.in, q.out, nullptr);
    }
  }
  if (!ctx->pending.on) return;
  const qnn_ctx_s::Pending p = ctx->pending;
  ctx->pending = {};
  p.g->pins--;
  p.u->pins--;
  run_int4(ctx, p.g, p.u, I4_SWIGLU, p.x, p.h, 1, p.in, p.out, nullptr);
}

bool mlp_fusion_enabled() { return tuning().fuse_mlp != 0; }

// A gate/up SwiGLU launch gives each row the sums the two I4_STORE launches
// would (same steps per wave, slices and parts for every 16-row chunk), so
// the recorded triple stays bit-identical to the separate operations.
bool glu_plans_match(const I4Layout &l, int rows) {
  for (int r0 = 0; r0 < rows; r0 += 16) {
    const int m = std::min(16, rows - r0);
    const I4Plan a = int4_plan(l, m, I4_STORE), b = int4_plan(l, m, I4_SWIGLU);
    if (a.mt != b.mt || a.gsw != b.gsw || a.steps_per_slice != b.steps_per_slice || a.slices != b.slices ||
        a.tiles_per_wg != b.tiles_per_wg)
      return false;
  }
  return true;
}

// Completion flags of the single-launch kernels (fused MLP, one-token MoE):
// words 256 B apart that hold the epoch of the launch that last completed the
// block; zeroed when allocated, and epoch 0 is never a launch's.
void ensure_flags(qnn_ctx_s *ctx, size_t bytes) {
  if (bytes <= ctx->mlp_flag_bytes) return;
  sync(ctx);
  if (ctx->mlp_flags) (void)hipFree(ctx->mlp_flags);
  ctx->mlp_flags = nullptr;
  ctx->mlp_flag_bytes = 0;
  hip_check(hipMalloc(&ctx->mlp_flags, bytes), "completion flags");
  hip_check(hipMemsetAsync(ctx->mlp_flags, 0, bytes, ctx->stream), "completion flags");
  hip_check(hipStreamSynchronize(ctx->stream), "completion flags");
  ctx->mlp_flag_bytes = bytes;
}
unsigned next_epoch(qnn_ctx_s *ctx) {
  if (++ctx->mlp_epoch == 0) ctx->mlp_epoch = 1;
  return ctx->mlp_epoch;
}

// Launches the recorded SwiGLU and the down projection `d` (h -> y) as one
// kernel when the per-op plans allow it; false leaves the pending
// SwiGLU recorded.
bool try_fused_mlp(qnn_ctx_s *ctx, WeightEntry *d, float *y) {
  qnn_ctx_s::Pending &p = ctx->pending;
  const I4Layout &lg = p.g->i4, &ld = d->i4;
  if (lg.lanes != 1 || ld.lanes != 1 || p.in % 4 || p.out % 4) return false;
  // Its weight resources span whole matrices (32-bit offsets).
  if (std::max(lg.nib_bytes(), ld.nib_bytes()) > 0xFFFFFFFFull) return false;
  const I4Plan pg = int4_plan(lg, 1, I4_SWIGLU), pd = int4_plan(ld, 1, I4_STORE);
  if (pg.tiles_per_wg != 1 || pd.tiles_per_wg != 1 || pg.gsw > 8 || pd.gsw > 8) return false;
  const int grid = std::max(pg.grid, pd.grid);
  int &cap = ctx->mlp_cap[pg.gsw][pd.gsw];
  if (cap == 0) cap = std::max(-1, mlp_capacity(pg.gsw, pd.gsw, ctx->device));
  if (cap <= 0 || grid > cap) return false;
  const size_t pf_gu = size_t(2 * lg.blocks) * pg.slices * 64, pf_dn = size_t(ld.blocks) * pd.slices * 64;
  const size_t c_gu = size_t(lg.blocks) * kCounterStride, c_dn = size_t(ld.blocks) * kCounterStride;
  // Sized for the per-op pair too: a graph capture of the same sequence runs
  // it unfused, and a capture cannot grow the workspace.
  ensure_splitk(ctx, std::max({pf_gu + pf_dn, pg.partial_floats, pd.partial_floats}),
                std::max({c_gu + c_dn, pg.counters, pd.counters}));
  ensure_flags(ctx, size_t(lg.blocks) * 256);
  MlpLaunch a;
  a.lg = lg;
  a.ld = ld;
  a.gnib = p.g->dptr;
  a.gscl = static_cast<const uint8_t *>(p.g->dptr) + lg.nib_bytes();
  a.unib = p.u->dptr;
  a.uscl = static_cast<const uint8_t *>(p.u->dptr) + lg.nib_bytes();
  a.dnib = d->dptr;
  a.dscl = static_cast<const uint8_t *>(d->dptr) + ld.nib_bytes();
  a.x = p.x;
  a.h = p.h;
  a.y = y;
  a.hidden = p.in;
  a.inter = p.out;
  a.sps_gu = pg.steps_per_slice;
  a.slices_gu = pg.slices;
  a.sps_dn = pd.steps_per_slice;
  a.slices_dn = pd.slices;
  a.grid_dn = pd.grid;
  a.partial_gu = ctx->partial;
  a.partial_dn = ctx->partial + pf_gu;
  a.counters_gu = ctx->counters;
  a.counters_dn = ctx->counters + c_gu;
  a.flags = static_cast<unsigned *>(ctx->mlp_flags);
  a.epoch = next_epoch(ctx);
  a.err = ctx->error_flag;
  if (!mlp_launch(a, pg.gsw, pd.gsw, grid, ctx->stream)) return false;
  p.g->pins--;
  p.u->pins--;
  ctx->pending = {};
  ctx->st.mlp_fused++;
  return true;
}

// ---------------------------------------------------------------- Q8_0 multi-row GEMM
// Rows at which the MFMA GEMM replaces per-row matvecs (one weight pass per row).
int q8_gemm_min_rows() { return std::max(2, tuning().q8_gemm_min_rows); }

// The fp16 copy of a resident GGUF weight for the GEMM (k_h16_gemm), found or
// made on the device: a cache entry of its own (key + "/h16"), evicted like
// any other (its eviction is not reported).  A Q8_0 copy scales by the
// weight's own row exponents; a copy of any other encoding carries its row
// exponents after the values.  Null under graph capture when it does not
// exist yet (making it allocates).
WeightEntry *h16_entry(qnn_ctx_s *ctx, const WeightEntry *w) {
  const std::string key = w->key + "/h16";
  if (WeightEntry *h = lookup(ctx, key)) return h;
  if (ctx->capturing) return nullptr;
  const bool own_exp = w->gg.enc != QNN_WE_Q8_0;
  const size_t vbytes = q8_h16_bytes(w->gg.rows, w->gg.cols);
  auto *e = new WeightEntry();
  e->key = key;
  e->identity = w->identity;
  e->kind = WKind::Raw;
  e->derived = true;
  e->bytes = vbytes + (own_exp ? (size_t(w->gg.rows) * 4 + 255) / 256 * 256 : 0);
  e->source_bytes = 0;
  try {
    e->dptr = alloc_weight(ctx, e->bytes);
    if (own_exp) {
      int *ew = reinterpret_cast<int *>(static_cast<uint8_t *>(e->dptr) + vbytes);
      gguf_rowexp_launch(w->gg, w->dptr, ew, w->gg.rows, ctx->stream);
      gguf_expand_h16_launch(w->gg, w->dptr, ew, e->dptr, ctx->stream);
    } else {
      q8_expand_h16_launch(w->gg, w->dptr, e->dptr, ctx->stream);
    }
  } catch (...) {
    if (e->dptr) (void)hipFree(e->dptr);
    delete e;
    throw;
  }
  return insert(ctx, e);
}

// Rows per GEMM launch: the activation fragments (2 bytes per element, K
// padded to 64) stay below 4 GiB; QNN_GEMM_MAX_ROWS lowers it (tests).
int gemm_max_rows(int in_dim) {
  const size_t k_pad = (size_t(in_dim) + 63) / 64 * 64;
  size_t m = std::max<size_t>(128, 0xFFFFFFFFull / (k_pad * 2) / 128 * 128);
  if (tuning().gemm_max_rows > 0) m = std::min(m, size_t(tuning().gemm_max_rows));
  return int(std::min<size_t>(m, size_t(1) << 30));
}

// Multi-row GGUF projection.  From QNN_GEMM_H16 rows (Q8_0) or
// QNN_GGUF_GEMM_ROWS rows (the other encodings): k_h16_gemm over the weight's
// fp16 copy; otherwise, and under capture while no copy exists, a Q8_0 weight
// from q8_gemm_min_rows rows takes k_q8_gemm, which decodes its tiles.  False
// when neither applies: the caller then runs the matvec, up to kGGMaxTokens
// rows per pass.  (Measured with the GEMM's K-slices: at 8 rows the matvec is
// faster for Q4_K 4096 x 3584 (15.7 against 24.2 us) and Q6_K 3584 x 14336,
// even for Q2_K 14336 x 3584, slower for IQ2_XXS; from 16 rows the GEMM is
// faster for all of them.)
bool run_gguf_gemm(qnn_ctx_s *ctx, WeightEntry *w, const float *x, float *y, int rows, int in_dim, int out_dim) {
  const bool q8 = w->gg.enc == QNN_WE_Q8_0;
  const int from = q8 ? tuning().gemm_h16 : tuning().gguf_gemm_rows;
  // The GEMM kernels address the weight (its tiles, or its fp16 copy) and the
  // activation fragments with 32-bit buffer offsets: larger weights take the
  // matvec, and the caller passes at most gemm_max_rows rows.
  const size_t copy_bytes = q8_h16_bytes(w->gg.rows, w->gg.cols) + (size_t(w->gg.rows) * 4 + 255) / 256 * 256;
  if (from > 0 && rows >= from && copy_bytes <= 0xFFFFFFFFull) {
    w->op_pins++;  // making the copy may evict: not the weight it is made from
    WeightEntry *h = nullptr;
    try {
      h = h16_entry(ctx, w);
    } catch (...) {
      w->op_pins--;
      throw;
    }
    w->op_pins--;
    if (h) {
      const int *ew = q8 ? reinterpret_cast<const int *>(static_cast<const uint8_t *>(w->dptr) + w->gg.rowexp_off)
                         : reinterpret_cast<const int *>(static_cast<const uint8_t *>(h->dptr) +
                                                         q8_h16_bytes(w->gg.rows, w->gg.cols));
      const Q8GemmPlan p = q8_h16_plan(rows, in_dim, out_dim);
      // Small grids split K (the other encodings only: a Q8_0 copy's product
      // stays bit-identical to the decoding kernel's).
      const int ksplit = q8 ? 1 : h16_ksplit(p, out_dim);
      const size_t frag_off = 0, exp_off = (p.frag_bytes + 255) & ~size_t(255);
      const size_t part_off = (exp_off + p.exp_bytes + 255) & ~size_t(255);
      const size_t part_bytes = ksplit > 1 ? size_t(ksplit) * rows * out_dim * 4 : 0;
      uint8_t *ws = static_cast<uint8_t *>(ensure_work(ctx, part_off + part_bytes));
      q8_h16_gemm_launch(p, x, rows, in_dim, out_dim, ew, h->dptr, ws + frag_off,
                         reinterpret_cast<int *>(ws + exp_off), y, ctx->stream, ksplit,
                         reinterpret_cast<float *>(ws + part_off));
      ctx->st.gemm_h16++;
      return true;
    }
  }
  if (!q8 || rows < q8_gemm_min_rows() || w->gg.total > 0xFFFFFFFFull) return false;
  const Q8GemmPlan p = q8_gemm_plan(rows, in_dim, out_dim);
  const size_t frag_off = 0, exp_off = (p.frag_bytes + 255) & ~size_t(255);
  uint8_t *ws = static_cast<uint8_t *>(ensure_work(ctx, exp_off + p.exp_bytes));
  q8_gemm_launch(p, x, rows, in_dim, out_dim, w->gg, w->dptr, ws + frag_off, reinterpret_cast<int *>(ws + exp_off), y,
                 ctx->stream);
  return true;
}

// ---------------------------------------------------------------- GGUF projection
// nt (2..kGGMaxTokens) rows of x through one pass over the weight.
void run_gguf_mt(qnn_ctx_s *ctx, const WeightEntry *w, const float *x, float *y, int nt, int out_dim) {
  GGArgs a;
  a.l = w->gg;
  a.w = w->dptr;
  a.x = x;
  a.x_vec4 = (w->gg.cols % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  a.y = y;
  a.n = out_dim;
  a.tiles = w->gg.tiles;
  a.mode = GG_STORE;
  const int slices = (w->gg.units + 3) / 4;  // one unit per wave, four per workgroup
  ensure_splitk(ctx, slices > 1 ? size_t(a.tiles) * slices * 64 * kGGMaxTokens : 0, size_t(a.tiles) * kCounterStride);
  a.partial = ctx->partial;
  a.counters = ctx->counters;
  a.err = ctx->error_flag;
  gguf_matvec_mt_launch(a, slices, nt, ctx->stream);
}

void run_gguf(qnn_ctx_s *ctx, const WeightEntry *w, const WeightEntry *w2, int mode, const float *x, float *y,
              int out_dim, float *g_out, float *u_out) {
  GGArgs a;
  a.l = w->gg;
  a.w = w->dptr;
  a.w2 = w2 ? w2->dptr : nullptr;
  a.x = x;
  a.x_vec4 = (w->gg.cols % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  a.y = y;
  a.n = out_dim;
  a.tiles = mode >= GG_SWIGLU ? (out_dim + 31) / 32 : w->gg.tiles;
  a.mode = mode;
  a.g_out = g_out;
  a.u_out = u_out;
  int bw, slices;
  gguf_plan(w->gg, a.tiles, &bw, &slices);
  ensure_splitk(ctx, slices > 1 ? size_t(a.tiles) * slices * 64 : 0, size_t(a.tiles) * kCounterStride);
  a.partial = ctx->partial;
  a.counters = ctx->counters;
  a.err = ctx->error_flag;
  gguf_matvec_launch(a, bw, slices, ctx->stream);
}

}  // namespace
}  // namespace qnn

using namespace qnn;

extern "C" {

int qnn_last_error(char *buf, int len) {
  const int n = int(t_last_error.size());
  if (buf && len > 0) {
    const int c = std::min(n, len - 1);
    std::memcpy(buf, t_last_error.data(), c);
    buf[c] = 0;
  }
  return n;
}

int qnn_reload_tuning(void) {
  return guarded([&] {
    std::lock_guard<std::mutex> g(g_lock);
    reload_tuning();
    return QNN_OK;
  });
}

int qnn_phase_trace(qnn_ctx *ctx, uint64_t *dst, uint64_t count, uint64_t *copied) {
  return guarded([&] {
    check_ctx(ctx);
    if (!dst || !copied) fail(QNN_E_ARGUMENT, "phase trace buffer");
    sync(ctx);
    // [2048][16] words of the fused decode MLP, then of the one-token MoE kernel, then of k_attn_dma.
    constexpr uint64_t kWords = 2048 * 16;
    const int n = mlp_phase_read(dst, size_t(std::min(count, kWords)) * 8);
    if (n == -2) fail(QNN_E_NOT_SUPPORTED, "not a phase-trace build (libqnn_hip_trace.so)");
    if (n < 0) fail(QNN_E_INVALID_OP, "phase trace copy");
    int n2 = 0, n3 = 0;
    if (count > kWords) {
      n2 = moe_phase_read(dst + kWords, size_t(std::min(count - kWords, kWords)) * 8);
      if (n2 < 0) fail(QNN_E_INVALID_OP, "phase trace copy");
    }
    if (count > 2 * kWords) {
      n3 = attn_phase_read(dst + 2 * kWords, size_t(std::min(count - 2 * kWords, kWords)) * 8);
      if (n3 < 0) fail(QNN_E_INVALID_OP, "phase trace copy");
    }
    *copied = uint64_t(n) + uint64_t(n2) + uint64_t(n3);
    return QNN_OK;
  });
}

int qnn_stream_read(qnn_ctx *ctx, qnn_tensor *src, int count, qnn_tensor *dst) {
  return guarded([&] {
    check_ctx(ctx);
    check_tensor(ctx, src, count);
    check_tensor(ctx, dst, 1);
    if (count < 4 || count % 4) fail(QNN_E_ARGUMENT, "stream read count");
    misc_stream_read(src->ptr, size_t(count) * 4, reinterpret_cast<uint32_t *>(dst->ptr), ctx->stream);
    hip_check(hipGetLastError(), "stream read launch");
    return QNN_OK;
  });
}

int qnn_ctx_create(int device, uint64_t weight_cache_bytes, qnn_ctx **out) {
  return guarded([&] {
    if (!out) fail(QNN_E_ARGUMENT, "out");
    std::lock_guard<std::mutex> g(g_lock);
    // Context.Implementation.inc:14-17: one resident context per process.
    if (g_ctx) fail(QNN_E_INVALID_OP, "a resident HIP context already exists");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
      (void)hipGetLastError();
      fail(QNN_E_NOT_SUPPORTED, "no HIP device available");
    }
    if (device < 0 || device >= n) fail(QNN_E_ARGUMENT, "device index");
    hip_check(hipSetDevice(device), "hipSetDevice");
    reload_tuning();  // the QNN_* switches, read once here rather than per launch
    try {
      noalloc_scratch_init(device);  // the static scratch's address on this device, once
    } catch (const Error &) {
      // only qnn_int4_linear_noalloc needs it; that call reports the failure
    }
    auto *ctx = new qnn_ctx_s();
    ctx->device = device;
    ctx->owner = std::this_thread::get_id();
    try {
      hip_check(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
      hip_check(hipMalloc(&ctx->error_flag, 256), "error word");
      hip_check(hipMemsetAsync(ctx->error_flag, 0, 256, ctx->stream), "error word");
      hip_check(hipStreamSynchronize(ctx->stream), "error word");
      size_t free_b = 0, total_b = 0;
      hip_check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
      ctx->weight_limit = weight_cache_bytes ? weight_cache_bytes : uint64_t(double(free_b) * 0.85);
    } catch (...) {
      if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
      if (ctx->error_flag) (void)hipFree(ctx->error_flag);
      delete ctx;
      throw;
    }
    g_ctx = ctx;
    *out = ctx;
    return QNN_OK;
  });
}

int qnn_ctx_destroy(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    destroy_prefetch(ctx);
    for (auto &g : ctx->graphs) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    for (auto *s : ctx->sets) {
      if (s->mem) (void)hipFree(s->mem);
      delete s;
    }
    for (auto &kv : ctx->weights) {
      (void)hipFree(kv.second->dptr);
      delete kv.second;
    }
    for (auto *t : ctx->tensors) {
      (void)hipFree(t->ptr);
      delete t;
    }
    for (auto &e : ctx->events)
      if (e) (void)hipEventDestroy(e);
    if (ctx->partial) (void)hipFree(ctx->partial);
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->work) (void)hipFree(ctx->work);
    if (ctx->staging) (void)hipFree(ctx->staging);
    if (ctx->readback) (void)hipHostFree(ctx->readback);
    if (ctx->mlp_flags) (void)hipFree(ctx->mlp_flags);
    (void)hipFree(ctx->error_flag);
    (void)hipStreamDestroy(ctx->stream);
    std::lock_guard<std::mutex> g(g_lock);
    g_ctx = nullptr;
    delete ctx;
    return QNN_OK;
  });
}

int qnn_get_status(qnn_ctx *ctx, qnn_status *out) {
  return guarded([&] {
    check_ctx(ctx, true);  // a query: recorded ops stay recorded
    if (!out) fail(QNN_E_ARGUMENT, "out");
    ctx->st.weight_bytes = ctx->weight_bytes;
    ctx->st.weight_limit = ctx->weight_limit;
    *out = ctx->st;
    return QNN_OK;
  });
}

// ---------------------------------------------------------------- tensors
int qnn_tensor_new(qnn_ctx *ctx, int count, qnn_tensor **out) {
  return guarded([&] {
    // Recorded ops stay recorded: the engine creates each output right before
    // the projection that writes it (Work.New, QwenHybrid.pas:542, :700), and a
    // new tensor cannot alias a recorded op's buffers (Recycle settles them).
    check_ctx(ctx, true);
    if (!out) fail(QNN_E_ARGUMENT, "out");
    *out = new_tensor(ctx, count);
    return QNN_OK;
  });
}

int qnn_recycle(qnn_ctx *ctx, qnn_tensor **tensor) {
  return guarded([&] {
    check_ctx(ctx);
    if (!tensor || !*tensor) return QNN_OK;
    check_tensor(ctx, *tensor);
    (*tensor)->live = false;
    *tensor = nullptr;
    return QNN_OK;
  });
}

int qnn_scratch(qnn_ctx *ctx, int slot, int count, qnn_tensor **out) {
  return guarded([&] {
    check_ctx(ctx);
    if (slot < 0 || slot > 3 || !out) fail(QNN_E_ARGUMENT, "Resident scratch slot");
    if (!ctx->scratch[slot] || ctx->scratch[slot]->count < count) {
      if (ctx->scratch[slot]) ctx->scratch[slot]->live = false;
      ctx->scratch[slot] = new_tensor(ctx, count);
    }
    *out = ctx->scratch[slot];
    return QNN_OK;
  });
}

int qnn_upload_raw(qnn_ctx *ctx, const void *data, int count, qnn_tensor **out) {
  return guarded([&] {
    check_ctx(ctx);
    if (!data || !out) fail(QNN_E_ARGUMENT, "UploadRaw");
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "upload during graph capture");
    auto *t = new_tensor(ctx, count);
    hip_check(hipMemcpyAsync(t->ptr, data, size_t(count) * 4, hipMemcpyHostToDevice, ctx->stream), "upload");
    sync(ctx);
    *out = t;
    return QNN_OK;
  });
}

int qnn_download(qnn_ctx *ctx, qnn_tensor *t, void *dst, int count) {
  return guarded([&] {
    check_ctx(ctx);
    if (count == -1) count = t ? t->count : 0;
    if (count < 1) fail(QNN_E_ARGUMENT, "Empty resident download");
    check_tensor(ctx, t, count);
    if (!dst) fail(QNN_E_ARGUMENT, "Resident download");
    // Data and the error word land in one pinned buffer; the caller's memory is
    // written only when no error was flagged (Context.Implementation.inc:745-756).
    const size_t bytes = size_t(count) * 4;
    if (ctx->readback_bytes < bytes + 4) {
      if (ctx->readback) (void)hipHostFree(ctx->readback);
      ctx->readback = nullptr;
      ctx->readback_bytes = 0;
      hip_check(hipHostMalloc(&ctx->readback, bytes + 4, hipHostMallocDefault), "readback buffer");
      ctx->readback_bytes = bytes + 4;
    }
    auto *rb = static_cast<uint8_t *>(ctx->readback);
    hip_check(hipMemcpyAsync(rb, t->ptr, bytes, hipMemcpyDeviceToHost, ctx->stream), "download");
    hip_check(hipMemcpyAsync(rb + bytes, ctx->error_flag, 4, hipMemcpyDeviceToHost, ctx->stream), "error word");
    sync(ctx);
    release_flush_pins(ctx);
    ctx->st.readbacks++;
    int flag = 0;
    std::memcpy(&flag, rb + bytes, 4);
    if (flag) {
      hip_check(hipMemsetAsync(ctx->error_flag, 0, 4, ctx->stream), "error word reset");
      sync(ctx);
      if (flag & 2) fail(QNN_E_INVALID_OP, "single-launch kernel: a wait for data of the same launch timed out");
      if (flag & 8) fail(QNN_E_INVALID_OP, "Invalid GPU expert ID");  // LLM.MoE.pas:384-385
      if (flag & 16) fail(QNN_E_INVALID_OP, "MoE dispatch index outside its tensor");
      fail(QNN_E_INVALID_OP, "Resident GPU computation produced non-finite values");
    }
    std::memcpy(dst, rb, bytes);
    return QNN_OK;
  });
}

int qnn_copy(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, int count, int dst_offset, int src_offset) {
  return guarded([&] {
    check_ctx(ctx);
    if (count < 0 || dst_offset < 0 || src_offset < 0) fail(QNN_E_ARGUMENT, "Copy span");
    check_tensor(ctx, dst, int64_t(dst_offset) + count);
    check_tensor(ctx, src, int64_t(src_offset) + count);
    if (count)
      hip_check(hipMemcpyAsync(dst->ptr + dst_offset, src->ptr + src_offset, size_t(count) * 4,
                               hipMemcpyDeviceToDevice, ctx->stream),
                "copy");
    return QNN_OK;
  });
}

int qnn_flush(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx);
    sync(ctx);
    release_flush_pins(ctx);
    return QNN_OK;
  });
}

int qnn_tensor_count(const qnn_tensor *t) { return t ? t->count : -1; }
void *qnn_tensor_device_ptr(const qnn_tensor *t) { return t ? t->ptr : nullptr; }

// ---------------------------------------------------------------- residency
static WeightEntry *acquire_matrix(qnn_ctx_s *ctx, const qnn_weight *w, int rows, int cols) {
  check_weight_desc(w);
  if (is_gguf(w->encoding)) return acquire_gguf(ctx, w, rows, cols);
  if (w->dtype == QNN_DT_U8) {
    // Native INT4: cols is the stored row width Int4RowBytes(K); recover K from shape.
    const int k = (cols / 20) * 32;
    if (qnn_int4_row_bytes(k) != cols) fail(QNN_E_ARGUMENT, "INT4 row width is not a multiple of 20 bytes");
    return acquire_int4(ctx, w, rows, k);
  }
  // F32 / BF16 matrices [rows, cols] (the router, RetainRouters LLM.MoE.pas:190-194).
  if (w->dtype == QNN_DT_F32 || w->dtype == QNN_DT_BF16) return acquire_raw(ctx, w, int64_t(rows) * cols);
  fail(QNN_E_NOT_SUPPORTED, "only packed INT4, GGUF, F32 and BF16 matrices are resident in the HIP backend");
}

int qnn_retain_weight(qnn_ctx *ctx, const qnn_weight *w, int rows, int cols) {
  return guarded([&] {
    check_ctx(ctx);
    WeightEntry *e = acquire_matrix(ctx, w, rows, cols);
    // RetainWeight (Context.Implementation.inc:361-387): pinned for the context's
    // lifetime; retaining an entry twice keeps one pin.
    if (std::find(ctx->retained.begin(), ctx->retained.end(), e) != ctx->retained.end()) return QNN_OK;
    ctx->retained.push_back(e);
    e->pins++;
    ctx->retained_bytes += e->bytes;
    return QNN_OK;
  });
}

int qnn_preload_weights(qnn_ctx *ctx, const qnn_weight *ws, int n, uint64_t staging_limit) {
  return guarded([&] {
    check_ctx(ctx);
    (void)staging_limit;
    if (n < 0 || (n > 0 && !ws)) fail(QNN_E_ARGUMENT, "PreloadWeights");
    // Every preloaded entry stays pinned until the next Flush or Download, so a
    // later acquisition in the same batch cannot evict it (Context.API.inc:85-86).
    for (int i = 0; i < n; ++i) {
      WeightEntry *e = acquire_matrix(ctx, &ws[i], int(ws[i].shape0), int(ws[i].shape1));
      e->pins++;
      ctx->flush_pins.push_back(e);
    }
    return QNN_OK;
  });
}

int qnn_is_weight_resident(qnn_ctx *ctx, const qnn_weight *w, int rows, int cols, int *resident) {
  return guarded([&] {
    check_ctx(ctx, true);  // a query: recorded ops stay recorded
    check_weight_desc(w);
    if (!resident) fail(QNN_E_ARGUMENT, "out");
    std::string key;
    if (is_gguf(w->encoding)) key = weight_key("gg", w, gguf_weight_bytes(w, rows, cols));
    else if (w->dtype == QNN_DT_F32 || w->dtype == QNN_DT_BF16)
      key = weight_key("raw", w, uint64_t(rows) * cols * (w->dtype == QNN_DT_F32 ? 4 : 2));
    else key = weight_key("i4", w, uint64_t(rows) * cols);
    *resident = ctx->weights.count(key) ? 1 : 0;
    return QNN_OK;
  });
}

int qnn_weight_batch_capacity(qnn_ctx *ctx, uint64_t *bytes) {
  return guarded([&] {
    check_ctx(ctx, true);  // a query: recorded ops stay recorded
    if (!bytes) fail(QNN_E_ARGUMENT, "out");
    // WeightBatchCapacity (Context.Implementation.inc:421-429): the cache limit less the retained bytes.
    *bytes = ctx->weight_limit - std::min(ctx->weight_limit, ctx->retained_bytes);
    return QNN_OK;
  });
}

// ---------------------------------------------------------------- ops
int qnn_int4_linear(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int rows, int in_dim,
                    int out_dim) {
  return guarded([&] {
    check_ctx(ctx, true);
    try {
      // Int4Linear validation (Context.Implementation.inc:1091-1104).
      if (rows < 1 || rows > 128 || in_dim < 1 || out_dim < 1 || src == dst || int64_t(rows) * out_dim > 0x7fffffff)
        fail(QNN_E_ARGUMENT, "Invalid packed INT4 projection");
      check_tensor(ctx, src, int64_t(rows) * in_dim);
      check_tensor(ctx, dst, int64_t(rows) * out_dim);
      OpPins pin;
      WeightEntry *e = pin(acquire_int4(ctx, w, out_dim, in_dim));
      const qnn_ctx_s::Pending &p = ctx->pending;
      // The down projection of a recorded SwiGLU: one launch for the MLP.
      const bool fused = p.on && rows == 1 && src->ptr == p.h && in_dim == p.out && out_dim == p.in &&
                         dst->ptr != p.h && try_fused_mlp(ctx, e, dst->ptr);
      // Several rows: recorded to meet a following GO_SWIGLU (gate, up).
      qnn_ctx_s::PendingRows &q = ctx->prows;
      if (!fused && rows >= 2 && !ctx->capturing && mlp_fusion_enabled() && in_dim % 4 == 0 &&
          glu_plans_match(e->i4, rows)) {
        // Sized now (its own launch and the gate/up SwiGLU launch it may join),
        // so that launching it never allocates.
        size_t pf = 0, nc = 0;
        for (int r0 = 0; r0 < rows; r0 += 16) {
          const I4Plan a = int4_plan(e->i4, std::min(16, rows - r0), I4_STORE);
          const I4Plan b = int4_plan(e->i4, std::min(16, rows - r0), I4_SWIGLU);
          pf = std::max({pf, a.partial_floats, b.partial_floats});
          nc = std::max({nc, a.counters, b.counters});
        }
        ensure_splitk(ctx, pf, nc);
        if (q.count == 1 && q.x == src->ptr && q.rows == rows && q.in == in_dim && q.out == out_dim &&
            dst->ptr != q.y[0] && e->i4.rows == q.e[0]->i4.rows && e->i4.cols == q.e[0]->i4.cols &&
            e->i4.lanes == q.e[0]->i4.lanes) {
          e->pins++;
          q.e[1] = e;
          q.y[1] = dst->ptr;
          q.count = 2;
        } else {
          settle_pending(ctx);
          e->pins++;
          q.count = 1;
          q.e[0] = e;
          q.y[0] = dst->ptr;
          q.x = src->ptr;
          q.rows = rows;
          q.in = in_dim;
          q.out = out_dim;
        }
      } else if (!fused) {
        settle_pending(ctx);
        run_int4(ctx, e, nullptr, I4_STORE, src->ptr, dst->ptr, rows, in_dim, out_dim, nullptr);
      }
    } catch (...) {
      settle_pending(ctx);
      throw;
    }
    ctx->st.gemm_calls++;
    ctx->st.int4_calls++;
    return QNN_OK;
  });
}

int qnn_int4_linear_noalloc(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int rows, int in_dim,
                            int out_dim) {
  return guarded([&] {
    check_ctx(ctx, true);
    // Recorded calls sized their workspace when they were recorded, so
    // launching them here allocates nothing either.
    settle_pending(ctx);
    // Int4Linear validation (Context.Implementation.inc:1091-1104), plus the
    // limits of this variant.
    if (rows < 1 || rows > 128 || in_dim < 1 || out_dim < 1 || src == dst || int64_t(rows) * out_dim > 0x7fffffff)
      fail(QNN_E_ARGUMENT, "Invalid packed INT4 projection");
    if (in_dim % 4 != 0)
      fail(QNN_E_ARGUMENT, "the no-allocation INT4 projection needs an input width that is a multiple of 4");
    check_tensor(ctx, src, int64_t(rows) * in_dim);
    check_tensor(ctx, dst, int64_t(rows) * out_dim);
    check_weight_desc(w);
    const int rb = qnn_int4_row_bytes(in_dim);
    if (w->dtype != QNN_DT_U8 || w->encoding != QNN_WE_NATIVE || w->offset != 0 || rb < 0 || w->shape0 != out_dim ||
        w->shape1 != rb || int64_t(out_dim) * rb > w->size)
      fail(QNN_E_ARGUMENT, "Invalid packed INT4 projection");
    WeightEntry *e = lookup(ctx, weight_key("i4", w, uint64_t(out_dim) * rb));
    if (!e)
      fail(QNN_E_INVALID_OP,
           "weight not resident: the no-allocation projection does not upload (RetainWeight or PreloadWeights it first)");
    auto *base = static_cast<uint8_t *>(noalloc_scratch(ctx->device));
    if (!base) fail(QNN_E_INVALID_OP, "the static scratch of the no-allocation projection is not available on this device");
    for (int r0 = 0; r0 < rows; r0 += 16) {
      const I4Plan p = int4_plan(e->i4, std::min(16, rows - r0), I4_STORE);
      if (p.partial_floats * 4 > kNoAllocPartialBytes || p.counters * 4 > kNoAllocCounterBytes)
        fail(QNN_E_RANGE, "INT4 projection too large for the no-allocation scratch (7 MiB of partial sums, "
                          "1 MiB of tickets); use qnn_int4_linear");
    }
    FixedWs ws;
    ws.partial = reinterpret_cast<float *>(base);
    ws.counters = reinterpret_cast<unsigned *>(base + kNoAllocPartialBytes);
    OpPins pin;
    pin(e);
    run_int4(ctx, e, nullptr, I4_STORE, src->ptr, dst->ptr, rows, in_dim, out_dim, nullptr, nullptr, nullptr, &ws);
    ctx->st.gemm_calls++;
    ctx->st.int4_calls++;
    return QNN_OK;
  });
}

int qnn_int4_linear_accumulate(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, qnn_tensor *probabilities,
                               const qnn_weight *w, int in_dim, int out_dim, int prob_index) {
  return guarded([&] {
    check_ctx(ctx);
    // Int4LinearAccumulate validation (Context.Implementation.inc:1064-1068).
    if (in_dim < 1 || out_dim < 1 || prob_index < 0 || dst == src || dst == probabilities)
      fail(QNN_E_ARGUMENT, "Invalid accumulated INT4 vector projection");
    check_tensor(ctx, dst, out_dim);
    check_tensor(ctx, src, in_dim);
    check_tensor(ctx, probabilities, int64_t(prob_index) + 1);
    OpPins pin;
    WeightEntry *e = pin(acquire_int4(ctx, w, out_dim, in_dim));
    run_int4(ctx, e, nullptr, I4_ACCUM, src->ptr, dst->ptr, 1, in_dim, out_dim, probabilities->ptr + prob_index);
    ctx->st.int4_calls++;
    return QNN_OK;
  });
}

int qnn_swiglu_vector(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *gate, const qnn_weight *up,
                      int in_dim, int out_dim) {
  return guarded([&] {
    check_ctx(ctx);
    check_tensor(ctx, src, in_dim);
    check_tensor(ctx, dst, out_dim);
    if (in_dim < 1 || out_dim < 1 || dst == src) fail(QNN_E_ARGUMENT, "Invalid fused SwiGLU dimensions");
    check_weight_desc(gate);
    check_weight_desc(up);
    // Implementation.inc:1017-1022: two GGUF weights (op 67), two native INT4
    // weights (op 68), or two native F32/BF16 weights in any mix (op 66); any
    // other pair is not handled, and the caller falls back.
    const bool gg = is_gguf(gate->encoding) && is_gguf(up->encoding);
    const bool i4 = gate->dtype == QNN_DT_U8 && up->dtype == QNN_DT_U8 && gate->encoding == QNN_WE_NATIVE &&
                    up->encoding == QNN_WE_NATIVE;
    const auto dense = [](const qnn_weight *w) {
      return w->encoding == QNN_WE_NATIVE && (w->dtype == QNN_DT_F32 || w->dtype == QNN_DT_BF16);
    };
    const bool fp = !gg && !i4 && dense(gate) && dense(up);
    if (!gg && !i4 && !fp) return QNN_NOT_HANDLED;
    const int width = i4 ? qnn_int4_row_bytes(in_dim) : in_dim;
    if (gate->shape0 != out_dim || up->shape0 != out_dim || gate->shape1 != width || up->shape1 != width)
      fail(QNN_E_ARGUMENT, "Invalid fused SwiGLU weight shape");
    const auto elem_bytes = [](const qnn_weight *w) { return uint64_t(w->dtype == QNN_DT_BF16 ? 2 : 4); };
    uint64_t pair = i4   ? uint64_t(2) * out_dim * width
                    : fp ? uint64_t(out_dim) * in_dim * (elem_bytes(gate) + elem_bytes(up))
                         : gguf_weight_bytes(gate, out_dim, in_dim) + gguf_weight_bytes(up, out_dim, in_dim);
    uint64_t capacity = 0;
    qnn_weight_batch_capacity(ctx, &capacity);
    if (pair > capacity) {  // Implementation.inc:1033-1034
      int ra = 0, rb = 0;
      qnn_is_weight_resident(ctx, gate, out_dim, width, &ra);
      qnn_is_weight_resident(ctx, up, out_dim, width, &rb);
      if (!(ra && rb)) return QNN_NOT_HANDLED;
    }
    OpPins pin;
    if (i4) {
      WeightEntry *eg = pin(acquire_int4(ctx, gate, out_dim, in_dim));
      WeightEntry *eu = pin(acquire_int4(ctx, up, out_dim, in_dim));
      if (mlp_fusion_enabled() && !ctx->capturing && eg->i4.lanes == 1 && in_dim % 4 == 0 && out_dim % 4 == 0) {
        // Recorded: launched with the next call (fused if that is the down
        // projection of this output).  Pinned until then; the workspace of
        // its own launch is sized now, so launching it never allocates.
        const I4Plan pp = int4_plan(eg->i4, 1, I4_SWIGLU);
        ensure_splitk(ctx, pp.partial_floats, pp.counters);
        eg->pins++;
        eu->pins++;
        ctx->pending.on = true;
        ctx->pending.g = eg;
        ctx->pending.u = eu;
        ctx->pending.x = src->ptr;
        ctx->pending.h = dst->ptr;
        ctx->pending.in = in_dim;
        ctx->pending.out = out_dim;
      } else {
        run_int4(ctx, eg, eu, I4_SWIGLU, src->ptr, dst->ptr, 1, in_dim, out_dim, nullptr);
      }
      ctx->st.int4_calls += 2;
    } else if (fp) {  // op 66: one pass over the gate and up rows
      WeightEntry *eg = pin(acquire_raw(ctx, gate, int64_t(out_dim) * in_dim));
      WeightEntry *eu = pin(acquire_raw(ctx, up, int64_t(out_dim) * in_dim));
      dense_swiglu_launch(eg->dptr, eg->raw_dtype == QNN_DT_BF16, eu->dptr, eu->raw_dtype == QNN_DT_BF16, src->ptr,
                          dst->ptr, out_dim, in_dim, ctx->stream);
    } else {
      WeightEntry *eg = pin(acquire_gguf(ctx, gate, out_dim, in_dim));
      WeightEntry *eu = pin(acquire_gguf(ctx, up, out_dim, in_dim));
      if (gate->encoding == up->encoding) {
        run_gguf(ctx, eg, eu, GG_SWIGLU, src->ptr, dst->ptr, out_dim);  // one weight stream (op 67)
      } else {  // encodings differ: two matvecs and the elementwise SwiGLU
        qnn_tensor_s *g = new_tensor(ctx, out_dim), *u = new_tensor(ctx, out_dim);
        run_gguf(ctx, eg, nullptr, GG_STORE, src->ptr, g->ptr, out_dim);
        run_gguf(ctx, eu, nullptr, GG_STORE, src->ptr, u->ptr, out_dim);
        misc_glu(dst->ptr, g->ptr, u->ptr, out_dim, out_dim, 0, 0, ctx->stream);
        g->live = false;
        u->live = false;
      }
      ctx->st.gguf_calls += 2;
    }
    ctx->st.gemm_calls += 2;
    return QNN_OK;
  });
}

int qnn_linear(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, const qnn_weight *scales,
               const qnn_weight *bias, int rows, int in_dim, int out_dim) {
  return guarded([&] {
    check_ctx(ctx, true);
    try {
      check_tensor(ctx, src, int64_t(rows) * in_dim);
      check_tensor(ctx, dst, int64_t(rows) * out_dim);
      if (rows < 1 || in_dim < 1 || out_dim < 1 || src == dst)
        fail(QNN_E_ARGUMENT, "Invalid resident linear dimensions/alias");
      check_weight_desc(w);
      if (scales && scales->data) fail(QNN_E_NOT_SUPPORTED, "INT8 ConvRot weights are not handled by the HIP backend");
      const bool has_bias = bias && bias->data;
      if (!is_gguf(w->encoding)) {
        // F32 / BF16 weights (the gemm pipeline with the bf16 flag, Implementation.inc:852-883).
        if (w->dtype != QNN_DT_F32 && w->dtype != QNN_DT_BF16)
          fail(QNN_E_NOT_SUPPORTED, "Linear handles GGUF, F32 and BF16 weights; native INT4 goes through Int4Linear");
        settle_pending(ctx);
        OpPins pin;
        WeightEntry *e = pin(acquire_raw(ctx, w, int64_t(out_dim) * in_dim));
        const int bf = e->raw_dtype == QNN_DT_BF16;
        if (rows == 1) dense_matvec_launch(e->dptr, bf, src->ptr, dst->ptr, out_dim, in_dim, ctx->stream);
        else dense_gemm_launch(e->dptr, bf, src->ptr, dst->ptr, rows, out_dim, in_dim, ctx->stream);
        if (has_bias) {
          WeightEntry *b = pin(acquire_raw(ctx, bias, out_dim));
          misc_bias_add(dst->ptr, b->dptr, b->raw_dtype == QNN_DT_BF16, rows, out_dim, ctx->stream);
        }
        ctx->st.gemm_calls++;
        return QNN_OK;
      }
      OpPins pin;
      WeightEntry *e = pin(acquire_gguf(ctx, w, out_dim, in_dim));
      if (rows == 1 && !has_bias && !ctx->capturing && linear_grouping_enabled()) {
        // Recorded: launched with the next calls on the same input as one kernel.
        record_linear(ctx, e, src->ptr, dst->ptr, out_dim);
      } else {
        settle_pending(ctx);
        const int chunk = gemm_max_rows(in_dim);
        for (int r0 = 0; r0 < rows; r0 += chunk) {
          const int rr = std::min(chunk, rows - r0);
          const float *xs = src->ptr + size_t(r0) * in_dim;
          float *ys = dst->ptr + size_t(r0) * out_dim;
          if (rr >= 2 && run_gguf_gemm(ctx, e, xs, ys, rr, in_dim, out_dim)) continue;
          // The matvec (op 65): up to kGGMaxTokens rows per pass over the weight.
          for (int r = 0; r < rr; r += kGGMaxTokens) {
            const int nt = std::min(kGGMaxTokens, rr - r);
            if (nt == 1 || tuning().gg_mt == 0) {
              for (int t = r; t < r + nt; ++t)
                run_gguf(ctx, e, nullptr, GG_STORE, xs + size_t(t) * in_dim, ys + size_t(t) * out_dim, out_dim);
            } else {
              run_gguf_mt(ctx, e, xs + size_t(r) * in_dim, ys + size_t(r) * out_dim, nt, out_dim);
            }
          }
        }
        if (has_bias) {
          WeightEntry *b = pin(acquire_raw(ctx, bias, out_dim));
          misc_bias_add(dst->ptr, b->dptr, b->raw_dtype == QNN_DT_BF16, rows, out_dim, ctx->stream);
        }
      }
    } catch (...) {
      settle_pending(ctx);
      throw;
    }
    ctx->st.gemm_calls++;
    ctx->st.gguf_calls++;
    return QNN_OK;
  });
}

int qnn_vector_linear(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int in_dim, int out_dim) {
  return guarded([&] {
    check_ctx(ctx);
    // VectorLinear validation (Context.Implementation.inc:982-985).
    check_tensor(ctx, src, in_dim);
    check_tensor(ctx, dst, out_dim);
    check_weight_desc(w);
    if (in_dim < 1 || out_dim < 1 || src == dst || (w->dtype != QNN_DT_F32 && w->dtype != QNN_DT_BF16))
      fail(QNN_E_ARGUMENT, "Invalid resident vector projection");
    OpPins pin;
    WeightEntry *e = pin(acquire_raw(ctx, w, int64_t(out_dim) * in_dim));
    dense_matvec_launch(e->dptr, e->raw_dtype == QNN_DT_BF16, src->ptr, dst->ptr, out_dim, in_dim, ctx->stream);
    ctx->st.gemm_calls++;
    return QNN_OK;
  });
}

int qnn_upload(qnn_ctx *ctx, const qnn_weight *data, qnn_tensor **out) {
  return guarded([&] {
    check_ctx(ctx);
    // Upload(TMemoryBlock) (Context.Implementation.inc:700-705): F32 storage
    // only; Count = Size floats from element Offset (Common.pas:1234-1237, :1597-1605).
    if (!data || !out) fail(QNN_E_ARGUMENT, "Resident upload");
    if (data->dtype != QNN_DT_F32) fail(QNN_E_ARGUMENT, "Resident upload requires F32 storage");
    if (!data->data || data->offset < 0) fail(QNN_E_ARGUMENT, "Resident upload");
    if (data->size < 1 || data->size > 0x7fffffff) fail(QNN_E_RANGE, "resident tensor size");
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "upload during graph capture");
    auto *t = new_tensor(ctx, int(data->size));
    hip_check(hipMemcpyAsync(t->ptr, static_cast<const float *>(data->data) + data->offset, size_t(data->size) * 4,
                             hipMemcpyHostToDevice, ctx->stream),
              "upload");
    sync(ctx);
    *out = t;
    return QNN_OK;
  });
}

int qnn_set_weight_evicted(qnn_ctx *ctx, qnn_weight_evicted_fn fn, void *user) {
  return guarded([&] {
    check_ctx(ctx, true);
    ctx->on_evicted = fn;
    ctx->on_evicted_user = user;
    return QNN_OK;
  });
}

int qnn_q8_gemm_int8(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int rows, int in_dim,
                     int out_dim) {
  return guarded([&] {
    check_ctx(ctx);
    // Linear's validation (Context.Implementation.inc:826-829) for a Q8_0 weight.
    check_tensor(ctx, src, int64_t(rows) * in_dim);
    check_tensor(ctx, dst, int64_t(rows) * out_dim);
    if (rows < 1 || in_dim < 1 || out_dim < 1 || src == dst)
      fail(QNN_E_ARGUMENT, "Invalid resident linear dimensions/alias");
    check_weight_desc(w);
    if (w->encoding != QNN_WE_Q8_0) fail(QNN_E_NOT_SUPPORTED, "the int8-activation GEMM takes Q8_0 weights");
    OpPins pin;
    WeightEntry *e = pin(acquire_gguf(ctx, w, out_dim, in_dim));
    void *ws = ensure_work(ctx, q8_i8_workspace(rows, in_dim));
    q8_gemm_i8_launch(src->ptr, rows, in_dim, out_dim, e->gg, e->dptr, ws, dst->ptr, ctx->stream);
    ctx->st.gemm_calls++;
    ctx->st.gguf_calls++;
    return QNN_OK;
  });
}

// ---------------------------------------------------------------- asynchronous prefetch
int qnn_enable_weight_prefetch(qnn_ctx *ctx, uint64_t max_layer_bytes, int *enabled) {
  return guarded([&] {
    check_ctx(ctx);
    if (!enabled) fail(QNN_E_ARGUMENT, "out");
    *enabled = 0;
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    if (pf.enabled) {
      *enabled = max_layer_bytes <= pf.bytes;
      return QNN_OK;
    }
    // EnableWeightPrefetch (Context.Prefetch.inc:106-110).
    uint64_t capacity = 0;
    qnn_weight_batch_capacity(ctx, &capacity);
    const uint64_t padded = (max_layer_bytes + 255) & ~uint64_t(255);
    if (max_layer_bytes == 0 || max_layer_bytes > (uint64_t(512) << 20) || padded > capacity / 2) return QNN_OK;
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "prefetch set-up during graph capture");
    sync(ctx);
    try {
      hip_check(hipStreamCreateWithFlags(&pf.copy, hipStreamNonBlocking), "copy stream");
      for (auto &s : pf.slot) {
        hip_check(hipHostMalloc(&s.host, padded, hipHostMallocDefault), "prefetch host staging");
        hip_check(hipMalloc(&s.dev, padded), "prefetch device staging");
        hip_check(hipEventCreateWithFlags(&s.ready, hipEventDisableTiming), "prefetch event");
      }
    } catch (const Error &) {
      (void)hipGetLastError();
      destroy_prefetch(ctx);  // resource pressure changes scheduling, never results
      return QNN_OK;
    }
    pf.bytes = padded;
    pf.enabled = true;
    *enabled = 1;
    return QNN_OK;
  });
}

int qnn_begin_weight_prefetch(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx);  // launches what was recorded (Context.Prefetch.inc:153-161)
    if (!ctx->pf.enabled) fail(QNN_E_INVALID_OP, "Layer prefetch is disabled");
    return QNN_OK;
  });
}

int qnn_complete_weight_prefetch(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx);
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    // CompleteWeightPrefetch (Context.Prefetch.inc:388-405): wait for compute,
    // then release the batch it was using.
    sync(ctx);
    release_flush_pins(ctx);
    release_slot(ctx, pf.active);
    pf.active = -1;
    return QNN_OK;
  });
}

int qnn_prefetch_weights(qnn_ctx *ctx, const qnn_weight *ws, int n, int defer_join) {
  return guarded([&] {
    check_ctx(ctx);
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    if (!pf.enabled || pf.queued >= 0 || n < 1 || !ws) fail(QNN_E_INVALID_OP, "Invalid layer prefetch state");
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "prefetch during graph capture");
    std::vector<std::string> keys(n);
    std::vector<uint64_t> sizes(n);
    std::unordered_map<std::string, int> unique;
    uint64_t total = 0;
    for (int i = 0; i < n; ++i) {
      check_prefetch_matrix(&ws[i]);
      keys[i] = matrix_key(&ws[i]);
      sizes[i] = matrix_source_bytes(&ws[i]);
      if (unique.emplace(keys[i], i).second) total += (sizes[i] + 255) & ~uint64_t(255);
    }
    uint64_t capacity = 0;
    qnn_weight_batch_capacity(ctx, &capacity);
    if (total > pf.bytes || total > capacity / 2) fail(QNN_E_RANGE, "Layer prefetch exceeds the double-buffer budget");
    const int si = pf.next;
    qnn_ctx_s::PrefetchSlot &s = pf.slot[si];
    release_slot(ctx, si);
    const bool prepared = s.prepared_keys == keys;
    s.keys = keys;
    std::vector<bool> created(n, false);
    try {
      // Cache hits are pinned before any eviction (duplicates included).
      for (int i = 0; i < n; ++i) {
        auto it = ctx->weights.find(keys[i]);
        if (it == ctx->weights.end()) continue;
        WeightEntry *e = lookup(ctx, keys[i]);
        e->pins++;
        s.entries.push_back(e);
        created[i] = true;  // handled
      }
      uint64_t used = 0;
      std::unordered_map<std::string, bool> made;
      for (int i = 0; i < n; ++i) {
        if (created[i] || made.count(keys[i])) continue;
        const uint64_t off = prepared ? s.prepared_offsets[i] : used;
        WeightEntry *e = prefetch_entry(ctx, s, &ws[i], keys[i], sizes[i], off, prepared);
        s.entries.push_back(e);
        made[keys[i]] = true;
        used += (sizes[i] + 255) & ~uint64_t(255);
        ctx->st.weight_uploads++;
        ctx->st.weight_upload_bytes += sizes[i];
        ctx->st.async_weight_bytes += sizes[i];
      }
      hip_check(hipEventRecord(s.ready, pf.copy), "prefetch event");
      s.submitted = true;
    } catch (...) {
      (void)hipStreamSynchronize(pf.copy);
      s.submitted = false;
      // entries made here hold no valid data until the copies finish: drop them
      for (auto *e : s.entries) {
        e->pins--;
        if (e->ready == s.ready) {
          ctx->weights.erase(e->key);
          ctx->weight_bytes -= e->bytes;
          (void)hipFree(e->dptr);
          delete e;
        }
      }
      s.entries.clear();
      s.keys.clear();
      throw;
    }
    ctx->st.async_weight_batches++;
    s.prepared_keys.clear();
    s.prepared_offsets.clear();
    pf.queued = si;
    pf.next = 1 - si;
    if (!defer_join) return qnn_complete_weight_prefetch(ctx);
    return QNN_OK;
  });
}

int qnn_stage_weight_prefetch(qnn_ctx *ctx, const qnn_weight *ws, int n) {
  return guarded([&] {
    check_ctx(ctx, true);
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    if (!pf.enabled || pf.queued < 0) fail(QNN_E_INVALID_OP, "Host staging requires an uploaded next layer");
    if (n < 1 || !ws) fail(QNN_E_ARGUMENT, "StageWeightPrefetch");
    qnn_ctx_s::PrefetchSlot &s = pf.slot[pf.next];
    // Only the host buffer is reused here; its previous device weights stay
    // pinned until CompleteWeightPrefetch (Context.Prefetch.inc:322-327).
    if (s.submitted) {
      hip_check(hipEventSynchronize(s.ready), "prefetch slot");
      s.submitted = false;
    }
    s.prepared_keys.clear();
    s.prepared_offsets.clear();
    std::vector<std::string> keys(n);
    std::vector<uint64_t> offsets(n), sizes(n);
    std::unordered_map<std::string, int> unique;
    uint64_t total = 0;
    for (int i = 0; i < n; ++i) {
      check_prefetch_matrix(&ws[i]);
      keys[i] = matrix_key(&ws[i]);
      sizes[i] = matrix_source_bytes(&ws[i]);
      auto it = unique.find(keys[i]);
      if (it != unique.end()) {
        offsets[i] = offsets[it->second];
      } else {
        unique.emplace(keys[i], i);
        offsets[i] = total;
        total += (sizes[i] + 255) & ~uint64_t(255);
      }
    }
    if (total > pf.bytes) fail(QNN_E_RANGE, "Host-staged layer exceeds its buffer");
    for (auto &kv : unique)
      std::memcpy(static_cast<uint8_t *>(s.host) + offsets[kv.second], ws[kv.second].data, sizes[kv.second]);
    s.prepared_keys = keys;
    s.prepared_offsets = offsets;
    return QNN_OK;
  });
}

int qnn_activate_prefetched_weights(qnn_ctx *ctx, const qnn_weight *ws, int n, int *activated) {
  return guarded([&] {
    check_ctx(ctx, true);
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    if (!activated) fail(QNN_E_ARGUMENT, "out");
    *activated = 0;
    if (pf.queued < 0 || !ws) return QNN_OK;
    qnn_ctx_s::PrefetchSlot &s = pf.slot[pf.queued];
    if (n != int(s.keys.size())) return QNN_OK;
    for (int i = 0; i < n; ++i) {
      check_weight_desc(&ws[i]);
      if (matrix_key(&ws[i]) != s.keys[i]) return QNN_OK;
    }
    if (pf.active >= 0) fail(QNN_E_INVALID_OP, "Previous prefetched layer is still active");
    // Compute waits for the batch's copies (the reference's semaphore wait).
    hip_check(hipStreamWaitEvent(ctx->stream, s.ready, 0), "prefetch join");
    for (auto *e : s.entries)
      if (e->ready == s.ready) e->ready = nullptr;
    pf.active = pf.queued;
    pf.queued = -1;
    *activated = 1;
    return QNN_OK;
  });
}

int qnn_seal_weight_prefetch(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx, true);
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    if (pf.queued >= 0) fail(QNN_E_INVALID_OP, "Unused prefetched layer at forward completion");
    if (pf.active < 0) return QNN_OK;
    // The last layer's pins move to the next Flush/Download, as PreloadWeights'
    // do (Context.Prefetch.inc:421-438).
    qnn_ctx_s::PrefetchSlot &s = pf.slot[pf.active];
    for (auto *e : s.entries) ctx->flush_pins.push_back(e);
    s.entries.clear();
    s.keys.clear();
    pf.active = -1;
    return QNN_OK;
  });
}

int qnn_end_weight_prefetch(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx);
    qnn_ctx_s::Prefetch &pf = ctx->pf;
    sync(ctx);
    release_flush_pins(ctx);
    for (int i = 0; i < 2; ++i) {
      release_slot(ctx, i);
      pf.slot[i].prepared_keys.clear();
      pf.slot[i].prepared_offsets.clear();
    }
    pf.active = pf.queued = -1;
    return QNN_OK;
  });
}

int qnn_kernel(qnn_ctx *ctx, int op, int n, qnn_tensor *dst, qnn_tensor *a, qnn_tensor *b, qnn_tensor *c,
               const int *args, int nargs) {
  return guarded([&] {
    // A GLU may complete a recorded gate/up pair (checked below).
    const bool glu_pair = (op == QNN_GO_SWIGLU || op == QNN_GO_GEGLU) && ctx && ctx == g_ctx &&
                          (ctx->prows.count == 2 || ctx->lgroup.count == 2);
    check_ctx(ctx, glu_pair);
    auto arg = [&](int i) -> int {
      if (i >= nargs || !args) fail(QNN_E_ARGUMENT, "missing kernel argument");
      return args[i];
    };
    if (n < 0) fail(QNN_E_ARGUMENT, "kernel element count");
    switch (op) {
      case QNN_GO_FILL:
        check_tensor(ctx, dst, n);
        if (n) misc_fill(dst->ptr, n, uint32_t(arg(0)), ctx->stream);
        return QNN_OK;
      case QNN_GO_ADD: {
        const int cols = arg(0), stride = arg(1), doff = arg(3), soff = arg(4);
        float alpha;
        const int bits = arg(2);
        std::memcpy(&alpha, &bits, 4);
        if (cols < 1 || stride < cols || doff < 0 || soff < 0) fail(QNN_E_ARGUMENT, "GO_ADD geometry");
        check_tensor(ctx, a, int64_t(soff) + n);
        const int64_t rows = (int64_t(n) + cols - 1) / cols;
        check_tensor(ctx, dst, doff + (rows - 1) * stride + cols);
        if (n) misc_add(dst->ptr, a->ptr, n, cols, stride, alpha, doff, soff, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_SWIGLU:
      case QNN_GO_GEGLU: {
        const int inter = arg(0), inter_leaved = op == QNN_GO_SWIGLU ? arg(1) : 0;
        if (inter < 1) fail(QNN_E_ARGUMENT, "GLU width");
        check_tensor(ctx, dst, n);
        check_tensor(ctx, a, inter_leaved ? int64_t(n) * 2 : n);
        if (!inter_leaved) check_tensor(ctx, b, n);
        if (glu_pair && try_glu_group(ctx, op, n, inter_leaved, dst, a, b)) return QNN_OK;
        if (glu_pair) {
          const qnn_ctx_s::PendingRows q = ctx->prows;
          if (op == QNN_GO_SWIGLU && q.count == 2 && !inter_leaved && a->ptr == q.y[0] && b->ptr == q.y[1] &&
              inter == q.out && int64_t(n) == int64_t(q.rows) * q.out && dst->ptr != q.x) {
            ctx->prows = {};
            q.e[0]->pins--;
            q.e[1]->pins--;
            run_int4(ctx, q.e[0], q.e[1], I4_SWIGLU, q.x, dst->ptr, q.rows, q.in, q.out, nullptr, q.y[0], q.y[1]);
            ctx->st.glu_fused++;
            return QNN_OK;
          }
          settle_pending(ctx);
        }
        if (n) misc_glu(dst->ptr, a->ptr, inter_leaved ? nullptr : b->ptr, n, inter, inter_leaved,
                        op == QNN_GO_GEGLU, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_FINITE:
        check_tensor(ctx, a ? a : dst, n);
        if (n) misc_finite((a ? a : dst)->ptr, n, ctx->error_flag, ctx->stream);
        return QNN_OK;
      case QNN_GO_MOE_ROUTE: {
        const int rows = arg(0), experts = arg(1), k = arg(2), norm = arg(3);
        if (rows < 1 || experts < 1 || experts > 8192 || k < 1 || k > 64 || k > experts)
          fail(QNN_E_ARGUMENT, "GO_MOE_ROUTE geometry");
        check_tensor(ctx, a, int64_t(rows) * experts);
        check_tensor(ctx, dst, int64_t(rows) * k * 2);
        ctx->st.moe_calls++;
        if (rows == 1 && moe_route_j(experts) && !ctx->capturing && tuning().fuse_moe != 0 && dst != a) {
          ctx->proute = {true, a->ptr, dst->ptr, experts, k, norm};  // launched with the next call
          return QNN_OK;
        }
        misc_moe_route(dst->ptr, a->ptr, rows, experts, k, norm, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_MOE_GATHER: {
        const int hidden = arg(0), topk = arg(1), offset = arg(2);
        if (hidden < 1 || topk < 1 || offset < 0) fail(QNN_E_ARGUMENT, "GO_MOE_GATHER geometry");
        check_tensor(ctx, dst, n);
        check_tensor(ctx, b, int64_t(offset) + (n + hidden - 1) / hidden);
        check_tensor(ctx, a, 1);
        if (n) misc_moe_gather(dst->ptr, a->ptr, size_t(a->count), b->ptr, n, hidden, topk, offset, ctx->error_flag,
                               ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_MOE_SCATTER: {
        const int hidden = arg(0), topk = arg(1), offset = arg(2), route = arg(3), single = arg(4), pbase = arg(5);
        if (hidden < 1 || topk < 1 || offset < 0 || pbase < 0) fail(QNN_E_ARGUMENT, "GO_MOE_SCATTER geometry");
        check_tensor(ctx, a, n);
        check_tensor(ctx, dst, 1);
        check_tensor(ctx, c, int64_t(pbase) + 1);
        if (!single) check_tensor(ctx, b, int64_t(offset) + (n + hidden - 1) / hidden);
        if (n)
          misc_moe_scatter(dst->ptr, size_t(dst->count), a->ptr, single ? nullptr : b->ptr, c->ptr, size_t(c->count),
                           n, hidden, topk, offset, route, single, pbase, ctx->error_flag, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_SCALE: {
        // tensor.comp:309: dst = a * v0 + v1 (v1 defaults to 0, as an unset push constant).
        float mul, add = 0.0f;
        const int mb = arg(0), ab = nargs > 1 ? args[1] : 0;
        std::memcpy(&mul, &mb, 4);
        std::memcpy(&add, &ab, 4);
        check_tensor(ctx, a, n);
        check_tensor(ctx, dst, n);
        if (n) decode_scale(dst->ptr, a->ptr, n, mul, add, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_SOFTCAP: {
        float cap;
        const int cb = arg(0);
        std::memcpy(&cap, &cb, 4);
        check_tensor(ctx, a, n);
        check_tensor(ctx, dst, n);
        if (n) decode_softcap(dst->ptr, a->ptr, n, cap, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_LLM_CACHE_WRITE: {
        // Args [Rows, KvHeads, HeadDim, Capacity, Position] (LLM.pas:556-563).
        const int kvh = arg(1), dim = arg(2), cap = arg(3), pos = arg(4);
        if (kvh < 1 || dim < 1 || cap < 1 || pos < 0 || n % (int64_t(kvh) * dim) != 0)
          fail(QNN_E_ARGUMENT, "GO_LLM_CACHE_WRITE geometry");
        const int64_t rows = n / (int64_t(kvh) * dim);
        if (pos + rows > cap) fail(QNN_E_ARGUMENT, "GO_LLM_CACHE_WRITE: rows past the cache capacity");
        check_tensor(ctx, a, n);
        check_tensor(ctx, b, n);
        check_tensor(ctx, dst, 2 * int64_t(cap) * kvh * dim);
        if (n) decode_cache_write(dst->ptr, a->ptr, b->ptr, n, kvh, dim, cap, pos, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_LLM_ROPE: {
        // Args [Heads, HeadDim, Position, Theta bits] (LLM.pas:538-546); N = rows * heads * dim / 2.
        const int heads = arg(0), dim = arg(1), pos = arg(2), tb = arg(3);
        float theta;
        std::memcpy(&theta, &tb, 4);
        if (heads < 1 || dim < 2 || dim % 2 || pos < 0 || n % (int64_t(heads) * (dim / 2)) != 0 ||
            !(theta > 0.0f) || std::isinf(theta))
          fail(QNN_E_ARGUMENT, "GO_LLM_ROPE geometry");
        check_tensor(ctx, a, 2 * int64_t(n));
        check_tensor(ctx, dst, 2 * int64_t(n));
        if (n) decode_rope(dst->ptr, a->ptr, n, heads, dim, pos, theta, ctx->stream);
        return QNN_OK;
      }
      case QNN_GO_LLM_SEEN: {
        // Args [Vocab] (LLM.pas:643): flags[a[i]] |= 1 for ids below Vocab.
        const int vocab = arg(0);
        if (vocab < 1) fail(QNN_E_ARGUMENT, "GO_LLM_SEEN vocabulary");
        check_tensor(ctx, a, n);
        check_tensor(ctx, dst, vocab);
        if (n) decode_seen(dst->ptr, a->ptr, n, vocab, ctx->stream);
        return QNN_OK;
      }
    }
    fail(QNN_E_NOT_SUPPORTED, "op code not implemented by the HIP backend");
    return QNN_OK;
  });
}

int qnn_kernel_weights(qnn_ctx *ctx, int op, int n, qnn_tensor *dst, qnn_tensor *a, const qnn_weight *b,
                       const qnn_weight *c, const int *args, int nargs) {
  return guarded([&] {
    check_ctx(ctx);
    (void)n;
    if (op != QNN_GO_NORM) fail(QNN_E_NOT_SUPPORTED, "KernelWeights op not implemented by the HIP backend");
    if (!args || nargs < 8) fail(QNN_E_ARGUMENT, "GO_NORM needs 8 arguments");
    const int rows = args[0], dim = args[1], flags = args[2], soff = args[5], unit = args[6], epsb = args[7];
    if (rows < 1 || dim < 1 || soff < 0 || (flags & 2)) fail(QNN_E_ARGUMENT, "GO_NORM geometry (CHW layout not supported)");
    float eps = 1e-6f;
    if (epsb) std::memcpy(&eps, &epsb, 4);
    check_tensor(ctx, a, int64_t(soff) + int64_t(rows) * dim);
    check_tensor(ctx, dst, int64_t(soff) + int64_t(rows) * dim);
    OpPins pin;
    const void *gp = nullptr, *bp = nullptr;
    int gbf = 0, bbf = 0;
    if (!unit) {
      WeightEntry *g = pin(acquire_raw(ctx, b, dim));
      gp = g->dptr;
      gbf = g->raw_dtype == QNN_DT_BF16;
    }
    if ((flags & 1) && !(flags & 8)) {
      WeightEntry *be = pin(acquire_raw(ctx, c, dim));
      bp = be->dptr;
      bbf = be->raw_dtype == QNN_DT_BF16;
    }
    misc_norm(dst->ptr, a->ptr, gp, gbf, bp, bbf, rows, dim, flags, soff, unit, eps, ctx->stream);
    return QNN_OK;
  });
}

int qnn_gather(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *ids, const qnn_weight *w, const qnn_weight *scales, int rows,
               int dim, int vocab, int rotation) {
  return guarded([&] {
    check_ctx(ctx);
    if (rows < 1 || dim < 1 || vocab < 1) fail(QNN_E_ARGUMENT, "Gather geometry");
    check_tensor(ctx, dst, int64_t(rows) * dim);
    check_tensor(ctx, ids, rows);
    if (!w) fail(QNN_E_ARGUMENT, "Gather weight");
    if (rotation != 0) fail(QNN_E_NOT_SUPPORTED, "ConvRot weights are not handled by the HIP backend");
    OpPins pin;
    if (is_gguf(w->encoding)) {
      WeightEntry *e = pin(acquire_gguf(ctx, w, vocab, dim));
      gguf_gather_launch(e->gg, e->dptr, ids->ptr, dst->ptr, rows, vocab, ctx->stream);
      return QNN_OK;
    }
    if (w->dtype == QNN_DT_S8) {
      // Int8 rows with one F32 scale per row (AcquireInt8Weight).
      if (!scales) fail(QNN_E_ARGUMENT, "Gather: int8 rows need their scales");
      WeightEntry *e = pin(acquire_raw(ctx, w, int64_t(vocab) * dim, true));
      WeightEntry *sc = pin(acquire_raw(ctx, scales, vocab));
      if (sc->raw_dtype != QNN_DT_F32) fail(QNN_E_ARGUMENT, "Gather: int8 row scales must be F32");
      decode_gather(dst->ptr, ids->ptr, e->dptr, 2, static_cast<const float *>(sc->dptr), rows, dim, vocab,
                    ctx->stream);
      return QNN_OK;
    }
    WeightEntry *e = pin(acquire_raw(ctx, w, int64_t(vocab) * dim));
    decode_gather(dst->ptr, ids->ptr, e->dptr, e->raw_dtype == QNN_DT_BF16 ? 1 : 0, nullptr, rows, dim, vocab,
                  ctx->stream);
    return QNN_OK;
  });
}

int qnn_cached_attention(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *q, qnn_tensor *cache, int query_rows, int capacity,
                         int heads, int kv_heads, int dim, int position, int window, float softcap, float scale,
                         int masked) {
  return guarded([&] {
    check_ctx(ctx);
    // The argument rules of CachedAttention (Context.Implementation.inc:1194-1207).
    if (query_rows < 1 || query_rows > 65535 || capacity < 1 || position < 0 ||
        int64_t(position) + query_rows > capacity || heads < 1 || kv_heads < 1 || heads % kv_heads != 0 ||
        dim < 1 || dim > 1152 || window < 0 || !(softcap >= 0.0f) || std::isinf(softcap) || !(scale >= 0.0f) ||
        std::isinf(scale))
      fail(QNN_E_ARGUMENT, "Invalid resident cached attention");
    check_tensor(ctx, q, int64_t(query_rows) * heads * dim);
    check_tensor(ctx, dst, int64_t(query_rows) * heads * dim);
    check_tensor(ctx, cache, 2 * int64_t(capacity) * kv_heads * dim + (masked ? int64_t(query_rows) * capacity : 0));
    const AttnPlan p = attn_plan(query_rows, heads, kv_heads, dim, position, window);
    float *ws = p.part_floats ? static_cast<float *>(ensure_work(ctx, p.part_floats * 4)) : nullptr;
    attn_launch(q->ptr, cache->ptr, dst->ptr, ws, p, query_rows, capacity, heads, kv_heads, dim, position, window,
                softcap, scale, masked ? 1 : 0, ctx->stream);
    return QNN_OK;
  });
}

int qnn_sample_token(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *logits, qnn_tensor *seen, int vocab, int top_k,
                     float temperature, float top_p, float penalty, float uniform) {
  return guarded([&] {
    check_ctx(ctx);
    // The argument rules of SampleToken (Context.Implementation.inc:1143-1168).
    check_tensor(ctx, dst, 1);
    check_tensor(ctx, logits, vocab > 0 ? vocab : 1);
    check_tensor(ctx, seen, vocab > 0 ? vocab : 1);
    if (vocab < 1 || top_k < 1 || top_k > 64 || std::isnan(temperature) || std::isinf(temperature) ||
        temperature < 0 || std::isnan(top_p) || top_p <= 0 || top_p > 1 || std::isnan(penalty) ||
        std::isinf(penalty) || penalty <= 0 || std::isnan(uniform) || uniform < 0 || uniform >= 1 || dst == logits ||
        dst == seen)
      fail(QNN_E_ARGUMENT, "Invalid GPU token sampling arguments");
    const int k = temperature == 0.0f ? 1 : std::min(vocab, top_k);
    ensure_splitk(ctx, 0, 1);
    float *cand = static_cast<float *>(ensure_work(ctx, sample_workspace_floats(vocab, k) * 4));
    sample_launch(dst->ptr, logits->ptr, seen->ptr, cand, ctx->counters, vocab, k, temperature, top_p, penalty, uniform,
                  ctx->stream);
    return QNN_OK;
  });
}

int qnn_check_finite(qnn_ctx *ctx, qnn_tensor *t, int count) {
  return guarded([&] {
    check_ctx(ctx);
    if (count < 0) count = t ? t->count : 0;
    check_tensor(ctx, t, count);
    if (count) misc_finite(t->ptr, count, ctx->error_flag, ctx->stream);
    return QNN_OK;
  });
}

int qnn_dequantize(qnn_ctx *ctx, qnn_tensor *dst, const qnn_weight *w, int rows, int cols) {
  return guarded([&] {
    check_ctx(ctx);
    check_weight_desc(w);
    check_tensor(ctx, dst, int64_t(rows) * cols);
    OpPins pin;
    if (is_gguf(w->encoding)) {
      WeightEntry *e = pin(acquire_gguf(ctx, w, rows, cols));
      gguf_dequant_launch(e->gg, e->dptr, dst->ptr, ctx->stream);
    } else {
      WeightEntry *e = pin(acquire_int4(ctx, w, rows, cols));
      I4Layout l = e->i4;  // the resident layout depends on the group count only
      l.cols = cols;
      int4_dequant_launch(l, e->dptr, dst->ptr, ctx->stream);
    }
    return QNN_OK;
  });
}

// ---------------------------------------------------------------- routed experts
int qnn_expert_set_create(qnn_ctx *ctx, const qnn_weight *gate, const qnn_weight *up, const qnn_weight *down,
                          int experts, int hidden, int inter, qnn_expert_set **out) {
  return guarded([&] {
    check_ctx(ctx);
    if (!gate || !up || !down || !out || experts < 1 || experts > kMoEMaxExperts || hidden < 1 || inter < 1)
      fail(QNN_E_ARGUMENT, "Invalid expert set");
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "expert set creation during graph capture");
    const int rbh = qnn_int4_row_bytes(hidden), rbi = qnn_int4_row_bytes(inter);
    // Same descriptor rules as Int4Linear (Context.Implementation.inc:1093-1104).
    auto check = [&](const qnn_weight *w, int rows, int rb) {
      check_weight_desc(w);
      if (w->dtype != QNN_DT_U8 || w->encoding != QNN_WE_NATIVE || w->offset != 0 || rb < 0 || w->shape0 != rows ||
          w->shape1 != rb || int64_t(rows) * rb > w->size)
        fail(QNN_E_ARGUMENT, "Invalid packed INT4 expert projection");
    };
    for (int e = 0; e < experts; ++e) {
      check(&gate[e], inter, rbh);
      check(&up[e], inter, rbh);
      check(&down[e], hidden, rbi);
    }
    auto *set = new qnn_expert_set_s();
    set->experts = experts;
    set->hidden = hidden;
    set->inter = inter;
    set->gu = int4_layout(inter, hidden, true);
    set->dn = int4_layout(hidden, inter, true);
    const size_t gub = set->gu.bytes(), dnb = set->dn.bytes();
    set->bytes = size_t(experts) * (2 * gub + dnb);
    set->source_bytes = size_t(experts) * (2 * size_t(inter) * rbh + size_t(hidden) * rbi);
    try {
      if (hipMalloc(&set->mem, set->bytes) != hipSuccess) {
        (void)hipGetLastError();
        set->mem = nullptr;
        fail(QNN_E_RANGE, "expert set does not fit in device memory");
      }
      uint8_t *base = static_cast<uint8_t *>(set->mem);
      const size_t src_max = std::max(size_t(inter) * rbh, size_t(hidden) * rbi);
      for (int e = 0; e < experts; ++e) {
        const qnn_weight *ws[3] = {&gate[e], &up[e], &down[e]};
        uint8_t *dst[3] = {base + size_t(2 * e) * gub, base + size_t(2 * e + 1) * gub,
                           base + size_t(2 * experts) * gub + size_t(e) * dnb};
        for (int j = 0; j < 3; ++j) {
          const I4Layout &l = j < 2 ? set->gu : set->dn;
          const size_t nbytes = size_t(l.rows) * (j < 2 ? rbh : rbi);
          void *stg = ensure_staging(ctx, src_max);
          hip_check(hipMemcpyAsync(stg, ws[j]->data, nbytes, hipMemcpyHostToDevice, ctx->stream), "expert upload");
          int4_repack_launch(static_cast<const uint8_t *>(stg), l, dst[j], ctx->stream);
          sync(ctx);  // staging is reused by the next matrix
        }
      }
    } catch (...) {
      if (set->mem) (void)hipFree(set->mem);
      delete set;
      throw;
    }
    ctx->sets.push_back(set);
    *out = set;
    return QNN_OK;
  });
}

int qnn_expert_set_destroy(qnn_ctx *ctx, qnn_expert_set *set) {
  return guarded([&] {
    check_ctx(ctx);
    auto it = std::find(ctx->sets.begin(), ctx->sets.end(), set);
    if (it == ctx->sets.end()) fail(QNN_E_ARGUMENT, "unknown expert set");
    sync(ctx);  // queued launches may still read it
    if (set->mem) (void)hipFree(set->mem);
    ctx->sets.erase(it);
    delete set;
    return QNN_OK;
  });
}

int qnn_moe_experts(qnn_ctx *ctx, qnn_expert_set *set, qnn_tensor *dst, qnn_tensor *src, qnn_tensor *routes, int rows,
                    int topk) {
  return guarded([&] {
    check_ctx(ctx, true);
    // The route op recorded just before, for these routes: computed in the
    // one-token launch below if that launch happens; settled otherwise.
    qnn_ctx_s::PendingRoute fr = {};
    if (ctx->proute.on && routes && routes->ptr == ctx->proute.routes && rows == 1 &&
        std::find(ctx->sets.begin(), ctx->sets.end(), set) != ctx->sets.end() &&
        set->experts == ctx->proute.experts && topk == ctx->proute.k && src && src->ptr != ctx->proute.routes &&
        dst && dst->ptr != ctx->proute.logits) {
      fr = ctx->proute;
      ctx->proute = {};
    }
    settle_pending(ctx);  // every other recorded op runs before the experts read or write
    struct RouteGuard {  // an error below still runs the recorded route op
      qnn_ctx_s *ctx;
      qnn_ctx_s::PendingRoute &r;
      ~RouteGuard() {
        if (!r.on) return;
        try {
          misc_moe_route(r.routes, r.logits, 1, r.experts, r.k, r.normalize, ctx->stream);
        } catch (...) {  // a launch error surfaces at the next synchronising call
        }
      }
    } route_guard{ctx, fr};
    if (std::find(ctx->sets.begin(), ctx->sets.end(), set) == ctx->sets.end())
      fail(QNN_E_ARGUMENT, "unknown expert set");
    // TLLMMoE.forward geometry (LLM.MoE.pas:376-377) and the route op's limits.
    if (rows < 1 || rows > 128 || topk < 1 || topk > 64 || topk > set->experts || rows * topk > kMoEMaxRoutes)
      fail(QNN_E_ARGUMENT, "Invalid MoE forward geometry");
    check_tensor(ctx, src, int64_t(rows) * set->hidden);
    check_tensor(ctx, dst, int64_t(rows) * set->hidden);
    check_tensor(ctx, routes, int64_t(2) * rows * topk);
    if (dst == src || dst == routes) fail(QNN_E_ARGUMENT, "MoE output aliases an input");
    if (set->hidden % 4 != 0 || set->inter % 4 != 0)
      fail(QNN_E_NOT_SUPPORTED, "device MoE needs hidden and intermediate sizes that are multiples of 4");
    MoELaunch a;
    const uint8_t *base = static_cast<const uint8_t *>(set->mem);
    a.gu_stride = set->gu.bytes();
    a.dn_stride = set->dn.bytes();
    a.gate_up = base;
    a.down = base + size_t(2 * set->experts) * a.gu_stride;
    a.gu = set->gu;
    a.dn = set->dn;
    a.experts = set->experts;
    a.hidden = set->hidden;
    a.inter = set->inter;
    a.topk = topk;
    a.rows = rows;
    a.x = src->ptr;
    a.routes = routes->ptr;
    a.out = dst->ptr;
    const MoEPlanSizes p = moe_plan(a);
    const size_t n = size_t(rows) * topk;
    const size_t hfl = (n * set->inter + 63) / 64 * 64;
    float *w = static_cast<float *>(ensure_work(ctx, (hfl + n * set->hidden) * 4));
    a.h = w;
    a.y = w + hfl;
    ensure_splitk(ctx, p.partial_floats + p.plan_words, p.counters);
    a.partial = ctx->partial;
    a.counters = ctx->counters;
    a.plan = reinterpret_cast<int *>(ctx->partial + p.partial_floats);
    a.err = ctx->error_flag;
    ctx->st.int4_calls += 3;
    // One token: one launch (bit-identical to the two below) when every
    // workgroup of its grid can be resident; not under capture, where the
    // epoch baked into the launch would repeat on every replay.
    if (rows == 1 && !ctx->capturing && tuning().fuse_moe != 0) {
      const MoEDecodePlan d = moe_decode_plan(a, p);
      const int rj = fr.on && p.gsw == 8 ? moe_route_j(set->experts) : 0;
      if (d.ok) {
        int &cap = ctx->moe_cap[p.gsw][rj];
        if (cap == 0) cap = std::max(-1, moe_decode_capacity(p, rj, ctx->device));
        if (cap > 0 && d.grid <= cap) {
          ensure_splitk(ctx, d.partial_gu + d.partial_dn, d.counters_gu + d.counters_dn);
          ensure_flags(ctx, d.flag_bytes);
          a.partial = ctx->partial;
          a.partial_dn = ctx->partial + d.partial_gu;
          a.counters = ctx->counters;
          a.counters_dn = ctx->counters + d.counters_gu;
          a.flags = static_cast<unsigned *>(ctx->mlp_flags);
          a.epoch = next_epoch(ctx);
          if (rj) {
            a.logits = fr.logits;
            a.routes_out = fr.routes;
            a.normalize = fr.normalize;
          }
          if (moe_decode_launch(a, p, d, rj, ctx->stream)) {
            if (rj) {
              fr.on = false;  // computed by this launch
              ctx->st.moe_route_fused++;
            }
            ctx->st.moe_fused++;
            return QNN_OK;
          }
          hip_check(hipGetLastError(), "moe decode launch");
        }
      }
    }
    if (fr.on) {  // the routes first, then the two launches that read them
      fr.on = false;
      misc_moe_route(fr.routes, fr.logits, 1, fr.experts, fr.k, fr.normalize, ctx->stream);
    }
    moe_launch(a, p, ctx->stream);
    return QNN_OK;
  });
}


// ---------------------------------------------------------------- timing / graphs
int qnn_event_record(qnn_ctx *ctx, int slot) {
  return guarded([&] {
    check_ctx(ctx);
    if (slot < 0 || slot >= 64) fail(QNN_E_ARGUMENT, "event slot");
    if (!ctx->events[slot]) hip_check(hipEventCreate(&ctx->events[slot]), "hipEventCreate");
    hip_check(hipEventRecord(ctx->events[slot], ctx->stream), "hipEventRecord");
    return QNN_OK;
  });
}

int qnn_event_elapsed_ms(qnn_ctx *ctx, int a, int b, float *ms) {
  return guarded([&] {
    check_ctx(ctx);
    if (a < 0 || a >= 64 || b < 0 || b >= 64 || !ctx->events[a] || !ctx->events[b] || !ms)
      fail(QNN_E_ARGUMENT, "event slots");
    hip_check(hipEventSynchronize(ctx->events[b]), "hipEventSynchronize");
    hip_check(hipEventElapsedTime(ms, ctx->events[a], ctx->events[b]), "hipEventElapsedTime");
    return QNN_OK;
  });
}

int qnn_graph_begin(qnn_ctx *ctx) {
  return guarded([&] {
    check_ctx(ctx);
    if (ctx->capturing) fail(QNN_E_INVALID_OP, "capture already active");
    hip_check(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    ctx->capturing = true;
    ctx->capture_pins.clear();
    return QNN_OK;
  });
}

int qnn_graph_end(qnn_ctx *ctx, int *graph_id) {
  return guarded([&] {
    check_ctx(ctx);
    if (!ctx->capturing) fail(QNN_E_INVALID_OP, "no capture active");
    GraphRec g;
    ctx->capturing = false;
    const hipError_t ec = hipStreamEndCapture(ctx->stream, &g.graph);
    if (ec != hipSuccess) {
      for (auto *e : ctx->capture_pins) e->pins--;
      ctx->capture_pins.clear();
      hip_check(ec, "hipStreamEndCapture");
    }
    hip_check(hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    g.pinned = ctx->capture_pins;  // weights a graph reads stay resident
    ctx->capture_pins.clear();
    ctx->graphs.push_back(g);
    if (graph_id) *graph_id = int(ctx->graphs.size()) - 1;
    return QNN_OK;
  });
}

int qnn_graph_launch(qnn_ctx *ctx, int graph_id) {
  return guarded([&] {
    check_ctx(ctx);
    if (graph_id < 0 || graph_id >= int(ctx->graphs.size())) fail(QNN_E_ARGUMENT, "graph id");
    hip_check(hipGraphLaunch(ctx->graphs[graph_id].exec, ctx->stream), "hipGraphLaunch");
    return QNN_OK;
  });
}

void *qnn_stream(qnn_ctx *ctx) { return ctx ? ctx->stream : nullptr; }

}  // extern "C"
