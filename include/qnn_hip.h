/*
 * qnn_hip.h -- C ABI of libqnn_hip.so, the MI355X (gfx950) backend for
 * QuickNN's quantized-weight decode path.
 *
 * The library stands in for the Vulkan resident context TQNNGPUContext
 * (src/backends/vulkan/QuickNN.Vulkan.Context.API.inc:14-165) on the methods
 * the LLM engine in src/models calls for packed matvec, fused gate/up + SwiGLU
 * and routed-expert execution.  Every entry point is cdecl, takes plain
 * pointers and sizes, and returns a status code; the Object Pascal unit re-raises
 * the matching exception class.
 *
 * Conventions (as in the reference):
 *  - One context exists at a time; it is bound to the thread that created it
 *    (Context.Implementation.inc:10-18, :70-71).  Calls from another thread
 *    fail with QNN_E_INVALID_OP.
 *  - Ops record asynchronously on the context's HIP stream; qnn_flush and
 *    qnn_download wait (Context.Implementation.inc:399-419, :707-758).
 *  - Tensors are context-owned fp32 device buffers of `count` floats, pooled
 *    best-fit (Context.Implementation.inc:110-169).
 *  - Weights are host views described by qnn_weight (TMemoryBlock,
 *    src/core/QuickNN.Common.pas:135-155) and are copied into a device cache
 *    keyed by identity/dtype/encoding/offset/bytes (QuickNN.Vulkan.pas:641-662).
 *    Host memory need only stay valid during the call that uploads it.
 *    On upload the bytes are re-laid into the backend's tiled device layout;
 *    values and byte counts are unchanged.
 */
#ifndef QNN_HIP_H
#define QNN_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: exception classes of the reference ---- */
#define QNN_OK 0
#define QNN_NOT_HANDLED 1        /* TrySwiGLUVector returned False (caller falls back) */
#define QNN_NOT_FOUND 2          /* GetTensor returned nil (no tensor of that name) */
#define QNN_E_ARGUMENT (-1)      /* EArgumentException */
#define QNN_E_RANGE (-2)         /* ERangeError (budgets, device limits) */
#define QNN_E_NOT_SUPPORTED (-3) /* ENotSupportedException */
#define QNN_E_INVALID_OP (-4)    /* EInvalidOp (wrong thread, non-finite results, device failure) */
#define QNN_E_FORMAT (-5)        /* ESafeTensorError, EGGUFError (malformed or stale files) */
#define QNN_E_IO (-6)            /* EFOpenError / EFCreateError / EInOutError */

/* ---- TQNNDataType ordinals (src/core/QuickNN.Common.pas:71-90) ---- */
#define QNN_DT_UNDEF 0
#define QNN_DT_F16 1
#define QNN_DT_BF16 2
#define QNN_DT_F32 3
#define QNN_DT_S32 4
#define QNN_DT_S8 5
#define QNN_DT_U8 6
#define QNN_DT_F64 7
#define QNN_DT_BOOLEAN 8
#define QNN_DT_F8E5M2 9
#define QNN_DT_F8E4M3 10
#define QNN_DT_S4 11
#define QNN_DT_F4E2M1 14
#define QNN_DT_S16 16
#define QNN_DT_U16 17

/* ---- TQNNWeightEncoding ordinals (src/core/QuickNN.Common.pas:130-131) ---- */
#define QNN_WE_NATIVE 0
#define QNN_WE_Q8_0 1
#define QNN_WE_Q4_K 2
#define QNN_WE_Q6_K 3
#define QNN_WE_Q3_K 4
#define QNN_WE_Q5_K 5
#define QNN_WE_IQ4_NL 6
#define QNN_WE_IQ3_S 7
#define QNN_WE_IQ4_XS 8
#define QNN_WE_Q2_K 9
#define QNN_WE_IQ2_XXS 10
#define QNN_WE_IQ2_S 11
#define QNN_WE_Q2_0 12
#define QNN_WE_IQ3_XXS 13

/* ---- TSafeTensorType ordinals (src/io/QuickNN.SafeTensors.pas:34-77) ---- */
#define QNN_ST_UNKNOWN (-1)
#define QNN_ST_BOOL 0
#define QNN_ST_F4 1
#define QNN_ST_F6_E2M3 2
#define QNN_ST_F6_E3M2 3
#define QNN_ST_U8 4
#define QNN_ST_I8 5
#define QNN_ST_F8_E5M2 6
#define QNN_ST_F8_E4M3 7
#define QNN_ST_F8_E8M0 8
#define QNN_ST_I16 9
#define QNN_ST_U16 10
#define QNN_ST_F16 11
#define QNN_ST_BF16 12
#define QNN_ST_I32 13
#define QNN_ST_U32 14
#define QNN_ST_F32 15
#define QNN_ST_C64 16
#define QNN_ST_F64 17
#define QNN_ST_I64 18
#define QNN_ST_U64 19
#define QNN_ST_I4 20

/* ---- op codes accepted by qnn_kernel / qnn_kernel_weights
        (Context.API.inc:167-258) ---- */
#define QNN_GO_FILL 0
#define QNN_GO_NORM 2
#define QNN_GO_ADD 4
#define QNN_GO_SWIGLU 9
#define QNN_GO_FINITE 13
#define QNN_GO_SCALE 43
#define QNN_GO_LLM_CACHE_WRITE 44
#define QNN_GO_LLM_ROPE 45
#define QNN_GO_LLM_SEEN 48
#define QNN_GO_MOE_ROUTE 52
#define QNN_GO_MOE_GATHER 53
#define QNN_GO_MOE_SCATTER 54
#define QNN_GO_GEGLU 75
#define QNN_GO_SOFTCAP 76

/* OnWeightEvicted (Context.API.inc:164, TProc<IInterface>): called with the
 * evicted entry's WeightIdentity before its device memory is released
 * (QuickNN.Vulkan.pas:568-569).  It runs on the context's thread inside the
 * call that needed the room and must not call back into the context. */
typedef void (*qnn_weight_evicted_fn)(uint64_t identity, void *user);

typedef struct qnn_ctx_s qnn_ctx;       /* TQNNGPUContext */
typedef struct qnn_tensor_s qnn_tensor; /* TQNNGPUTensor: fp32 device buffer */
typedef struct qnn_expert_set_s qnn_expert_set;

/* TMemoryBlock view of a weight (src/core/QuickNN.Common.pas:135-155).
 * Native INT4: dtype U8, encoding NATIVE, shape [N, Int4RowBytes(K)], size in bytes, offset 0.
 * GGUF: dtype U8, encoding Q*, shape [N, K] in elements, size in elements,
 *       offset in elements (block-aligned); data points at element 0. */
typedef struct {
  uint64_t identity; /* WeightIdentity: non-zero; equal identity means the same immutable bytes */
  const void *data;  /* host storage base (element 0, before offset) */
  int64_t offset;    /* Offset */
  int64_t size;      /* Size */
  int64_t shape0;    /* Shape[0] */
  int64_t shape1;    /* Shape[1] */
  int32_t dtype;     /* TQNNDataType ordinal */
  int32_t encoding;  /* TQNNWeightEncoding ordinal */
} qnn_weight;

/* TQNNGPUStatus counters (src/backends/vulkan/QuickNN.Vulkan.pas:17-29). */
typedef struct {
  uint64_t gemm_calls, gguf_calls, int4_calls, moe_calls;
  uint64_t weight_uploads, weight_upload_bytes, weight_cache_hits, weight_cache_misses, weight_evictions;
  uint64_t readbacks, submissions;
  uint64_t weight_bytes, weight_limit, activation_bytes, activation_peak_bytes;
  uint64_t mlp_fused;      /* TrySwiGLUVector + Int4Linear pairs run as one launch (no reference counterpart) */
  uint64_t linear_grouped; /* one-row GGUF Linear calls that ran in a shared launch (no reference counterpart) */
  uint64_t moe_fused;      /* one-token qnn_moe_experts calls run as a single launch (no reference counterpart) */
  uint64_t moe_route_fused; /* of those, with the preceding GO_MOE_ROUTE computed in the launch (no reference counterpart) */
  uint64_t glu_fused;      /* multi-row Int4Linear gate + up + GO_SWIGLU triples run as one launch (no reference counterpart) */
  uint64_t async_weight_batches, async_weight_bytes; /* PrefetchWeights batches copied on the copy stream, and their bytes */
  uint64_t gemm_h16;       /* Q8_0 multi-row Linear calls run over the weight's pre-expanded fp16 copy (no reference counterpart) */
} qnn_status;

/* ---------------------------------------------------------------------------
 * Errors
 * ------------------------------------------------------------------------- */
/* Copies the calling thread's last error message; returns its length. */
int qnn_last_error(char *buf, int len);

/* ---------------------------------------------------------------------------
 * Context lifetime -- TQNNGPUContext.Create/Destroy (Context.Implementation.inc:14-80)
 * ------------------------------------------------------------------------- */
/* weight_cache_bytes = 0 selects 85% of the device's free memory. */
int qnn_ctx_create(int device, uint64_t weight_cache_bytes, qnn_ctx **out);
int qnn_ctx_destroy(qnn_ctx *ctx);
int qnn_get_status(qnn_ctx *ctx, qnn_status *out);
/* Re-reads the QNN_* tuning switches (experiment settings) from the
 * environment.  They are read once when a context is created, not per call;
 * this picks up a change made afterwards (tests and sweeps).  No reference
 * counterpart. */
int qnn_reload_tuning(void);
/* Diagnostic: per-workgroup phase timestamps (device real-time counter,
 * 100 MHz) of the fused decode-MLP kernel, as [2048 workgroups][16] words,
 * followed by the same for the one-token MoE kernel and for the LDS-streamed
 * cached-attention kernel, from a library built
 * with QNN_PHASE_TRACE (libqnn_hip_trace.so; the same kernels with
 * timestamps).  Waits for the context's work, copies up to `count` words into
 * dst, sets *copied and clears the timestamps.  QNN_E_NOT_SUPPORTED in the
 * ordinary build.  No reference counterpart. */
int qnn_phase_trace(qnn_ctx *ctx, uint64_t *dst, uint64_t count, uint64_t *copied);
/* Diagnostic: one plain streaming read of the first `count` floats of src
 * (count a multiple of 4), issued as the matvec kernels issue their weight
 * loads; dst (one float) is written only on a data-dependent condition.  Timed
 * with events, it gives the HBM stream floor of a buffer size.  No reference
 * counterpart. */
int qnn_stream_read(qnn_ctx *ctx, qnn_tensor *src, int count, qnn_tensor *dst);

/* ---------------------------------------------------------------------------
 * Resident tensors (Context.API.inc:79-106)
 * ------------------------------------------------------------------------- */
int qnn_tensor_new(qnn_ctx *ctx, int count, qnn_tensor **out);                 /* NewTensor */
int qnn_recycle(qnn_ctx *ctx, qnn_tensor **tensor);                            /* Recycle */
int qnn_scratch(qnn_ctx *ctx, int slot, int count, qnn_tensor **out);          /* Scratch */
int qnn_upload_raw(qnn_ctx *ctx, const void *data, int count, qnn_tensor **out); /* UploadRaw */
/* Upload(TMemoryBlock) (Context.Implementation.inc:700-705): F32 storage only
 * (else QNN_E_ARGUMENT); Size floats starting at element Offset. */
int qnn_upload(qnn_ctx *ctx, const qnn_weight *data, qnn_tensor **out);
int qnn_download(qnn_ctx *ctx, qnn_tensor *t, void *dst, int count);           /* Download (-1 = all) */
int qnn_copy(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, int count, int dst_offset, int src_offset); /* Copy */
int qnn_flush(qnn_ctx *ctx);                                                   /* Flush */
int qnn_tensor_count(const qnn_tensor *t);
void *qnn_tensor_device_ptr(const qnn_tensor *t);

/* ---------------------------------------------------------------------------
 * Weight residency (Context.API.inc:83-97; QuickNN.Vulkan.pas:551-740)
 * ------------------------------------------------------------------------- */
int qnn_retain_weight(qnn_ctx *ctx, const qnn_weight *w, int rows, int cols);  /* RetainWeight */
int qnn_preload_weights(qnn_ctx *ctx, const qnn_weight *ws, int n, uint64_t staging_limit); /* PreloadWeights */
int qnn_is_weight_resident(qnn_ctx *ctx, const qnn_weight *w, int rows, int cols, int *resident); /* IsWeightResident */
int qnn_weight_batch_capacity(qnn_ctx *ctx, uint64_t *bytes);                  /* WeightBatchCapacity */
/* OnWeightEvicted setter (Context.API.inc:164); fn = NULL clears it. */
int qnn_set_weight_evicted(qnn_ctx *ctx, qnn_weight_evicted_fn fn, void *user);

/* ---------------------------------------------------------------------------
 * Asynchronous layer prefetch (Context.API.inc:88-95, Context.Prefetch.inc:92-456).
 * Two slots, each a pinned host staging buffer and a device staging buffer of
 * max_layer_bytes; uploads run on a copy stream (host -> device copy, then the
 * repack into the weight cache) while the compute stream works.  The weights
 * of a PrefetchWeights batch are complete 2-D matrices (offset 0, size =
 * shape0 * shape1), pinned until the batch is released.  Any op that reads a
 * prefetched entry first makes the compute stream wait for its slot.
 * ------------------------------------------------------------------------- */
/* EnableWeightPrefetch: *enabled = 0 when max_layer_bytes is 0, above 512 MiB,
 * or above half the weight batch capacity (nothing is allocated then). */
int qnn_enable_weight_prefetch(qnn_ctx *ctx, uint64_t max_layer_bytes, int *enabled);
int qnn_begin_weight_prefetch(qnn_ctx *ctx);   /* BeginWeightPrefetch: launches recorded work */
/* PrefetchWeights: QNN_E_INVALID_OP unless enabled with no batch queued;
 * QNN_E_RANGE above the double-buffer budget.  defer_join = 0 also completes
 * (CompleteWeightPrefetch). */
int qnn_prefetch_weights(qnn_ctx *ctx, const qnn_weight *ws, int n, int defer_join);
/* StageWeightPrefetch: copies the next batch's host bytes into the free
 * slot's staging buffer now, so the following PrefetchWeights of the same
 * weights only starts the device copy. */
int qnn_stage_weight_prefetch(qnn_ctx *ctx, const qnn_weight *ws, int n);
int qnn_complete_weight_prefetch(qnn_ctx *ctx); /* CompleteWeightPrefetch: waits for compute, releases the active batch */
/* ActivatePrefetchedWeights: *activated = 1 when the queued batch holds
 * exactly these weights; it becomes the active batch and compute waits for it. */
int qnn_activate_prefetched_weights(qnn_ctx *ctx, const qnn_weight *ws, int n, int *activated);
int qnn_seal_weight_prefetch(qnn_ctx *ctx);    /* SealWeightPrefetch: active pins move to the next Flush */
int qnn_end_weight_prefetch(qnn_ctx *ctx);     /* EndWeightPrefetch: waits and releases both slots */

/* ---------------------------------------------------------------------------
 * Hot-path ops
 * ------------------------------------------------------------------------- */
/* Linear (Context.API.inc:117-122, Implementation.inc:813-899).  GGUF weights:
 * rows == 1 runs the packed matvec (op 65), rows > 1 the multi-row product
 * (gemm.comp): the fp16-MFMA GEMM for Q8_0 from 4 rows and for the other
 * encodings from 12 (over a cached fp16 copy of the weight), otherwise the
 * matvec up to 8 rows per pass over the weight.  F32 and BF16
 * weights [out_dim, in_dim] (the router and native-precision layers) run an
 * fp32 matvec (rows == 1) or fp32 GEMM (rows > 1); bf16 widens exactly.  One-row calls
 * without bias are recorded and launched by the next call on the context;
 * consecutive ones on the same src (up to 4; one encoding, or two K-quant
 * encodings) share one launch, each result identical to its own launch (QNN_GROUP_LINEAR=0 turns
 * this off); a group of exactly a gate and an up projection followed by
 * QNN_GO_GEGLU / QNN_GO_SWIGLU of their outputs runs as one gate/up launch
 * that also writes both outputs, identical to the separate ops.  bias (optional,
 * F32 or BF16 [out]) is added afterwards.  scales must be NULL (INT8 ConvRot
 * weights are outside this backend). */
int qnn_linear(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, const qnn_weight *scales,
               const qnn_weight *bias, int rows, int in_dim, int out_dim);

/* No counterpart in the reference: the benchmark's prefill GEMM for a Q8_0
 * weight [out_dim, in_dim], dst[r] = W src[r] for rows r, with the
 * activations quantised per 32-element block to int8 (d = max|x|/127 in fp32,
 * q = roundf(x / d)) and the products on the int8 matrix cores.  Block b adds
 * fma(float(S_b), dx * dw, acc) in ascending b, S_b the exact int32 block dot,
 * so results are reproducible bit for bit.  The quantisation moves results
 * about 5e-3 (normwise, N(0,1) activations) from the reference's fp32-
 * activation product; qnn_linear stays within 1e-3 of it. */
int qnn_q8_gemm_int8(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int rows, int in_dim,
                     int out_dim);

/* VectorLinear (Context.API.inc:130, Implementation.inc:969-1001): dst = W src for
 * an F32 or BF16 weight [out_dim, in_dim]; any other dtype is QNN_E_ARGUMENT.
 * The engine's router projection for one token (LLM.MoE.pas:363) and the
 * native-precision projections of LLM.pas:471, QwenHybrid.pas:548 and
 * Gemma2.pas:146. */
int qnn_vector_linear(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int in_dim, int out_dim);

/* Int4Linear (Context.API.inc:138-142, Implementation.inc:1080-1135):
 * 1 <= rows <= 128; weight U8/NATIVE [out_dim, Int4RowBytes(in_dim)], offset 0.
 * A multi-row call may be recorded and launched with the next call: two on
 * the same input followed by QNN_GO_SWIGLU of their outputs (the engine's
 * multi-row MLP) run as one gate/up SwiGLU launch that also writes both
 * outputs, bit-identical to the three separate operations. */
int qnn_int4_linear(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int rows, int in_dim,
                    int out_dim);

/* No counterpart in the reference.  Int4Linear for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments and results as
 * qnn_int4_linear (bit for bit), but it never uploads, records or allocates.
 *  - The weight must already be resident (RetainWeight / PreloadWeights /
 *    an earlier call); otherwise QNN_E_INVALID_OP.
 *  - in_dim must be a multiple of 4 (QNN_E_ARGUMENT), and the projection's
 *    split-K workspace must fit the library's fixed device scratch of 8 MiB
 *    per GPU (7 MiB partial sums, 1 MiB tickets), else QNN_E_RANGE.
 *  - Every call on a GPU shares that scratch; calls are ordered on the
 *    context's stream, so two of them that overlap on one GPU (for example a
 *    captured graph replayed on another stream during an eager call) race.
 *  - Calls recorded before it are launched first; they sized their own
 *    workspace when they were recorded. */
int qnn_int4_linear_noalloc(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *w, int rows,
                            int in_dim, int out_dim);

/* TrySwiGLUVector (Context.API.inc:132-133, Implementation.inc:1003-1056):
 * dst[o] = silu(gate.x)[o] * (up.x)[o].  Handles two GGUF weights (op 67),
 * two native INT4 weights (op 68) and two native F32/BF16 weights in any mix
 * (op 66, one pass over both rows).  Returns QNN_OK, or QNN_NOT_HANDLED
 * where the reference returns False (any other mix, or the pair does not fit
 * the weight budget and is not resident).  A native-INT4 pair is
 * recorded and launched by the next call on the context; when that call is
 * the qnn_int4_linear that reads dst (the MLP's down projection, one row),
 * both run as one launch with results identical to two (QNN_FUSE_MLP=0 turns
 * this off). */
int qnn_swiglu_vector(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, const qnn_weight *gate, const qnn_weight *up,
                      int in_dim, int out_dim);

/* Int4LinearAccumulate (Context.API.inc:134-135, Implementation.inc:1058-1078):
 * dst[o] += probabilities[prob_index] * (W src)[o]. */
int qnn_int4_linear_accumulate(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *src, qnn_tensor *probabilities,
                               const qnn_weight *w, int in_dim, int out_dim, int prob_index);

/* Kernel (Context.API.inc:110) for the hot-path ops:
 *   QNN_GO_FILL        args [bits]                       dst[i] = float(bits), i < n
 *   QNN_GO_ADD         args [cols, dst_stride, alpha_bits, dst_off, src_off]  (tensor.comp:221)
 *   QNN_GO_SWIGLU      args [I, interleaved]             (tensor.comp:228)
 *   QNN_GO_GEGLU       args [I, 0]                       (tensor.comp:228)
 *   QNN_GO_FINITE      args []                           same as qnn_check_finite
 *   QNN_GO_MOE_ROUTE   args [rows, experts, topk, normalize]   (moe.comp:25-50)
 *   QNN_GO_MOE_GATHER  args [hidden, topk, offset]             (moe.comp:124)
 *   QNN_GO_MOE_SCATTER args [hidden, topk, offset, route_index, single_row, prob_base] (moe.comp:125-126)
 *   QNN_GO_SCALE       args [mul_bits, add_bits = 0]     dst = a * mul + add (tensor.comp:309)
 *   QNN_GO_SOFTCAP     args [cap_bits]                   dst = cap * tanh(clamp(a / cap, -20, 20)) (tensor.comp:308)
 *   QNN_GO_LLM_ROPE    args [heads, dim, position, theta_bits]; n = rows * heads * dim / 2;
 *                      pairs (j, j + dim/2) of each head row rotated by
 *                      (position + row) * theta^(-2j/dim) (tensor.comp:318-327)
 *   QNN_GO_LLM_CACHE_WRITE args [rows, kv_heads, dim, capacity, position]; n = rows * kv_heads * dim;
 *                      dst = cache, a = K, b = V: K transposed [kv_heads][dim][capacity],
 *                      then V [kv_heads][capacity][dim] (tensor.comp:313-317)
 *   QNN_GO_LLM_SEEN    args [vocab]: dst[a[i]] |= 1 (token ids as raw bits) (tensor.comp:328)
 * a, b, c may be NULL where the op does not read them. */
int qnn_kernel(qnn_ctx *ctx, int op, int n, qnn_tensor *dst, qnn_tensor *a, qnn_tensor *b, qnn_tensor *c,
               const int *args, int nargs);

/* KernelWeights (Context.API.inc:111-116) for GO_NORM (tensor.comp:63-73):
 *   args [rows, dim, flags, 0, 0, src_offset, unit_gamma, eps_bits]; b = gamma (F32/BF16 [dim]). */
int qnn_kernel_weights(qnn_ctx *ctx, int op, int n, qnn_tensor *dst, qnn_tensor *a, const qnn_weight *b,
                       const qnn_weight *c, const int *args, int nargs);

/* Gather (Context.API.inc:147-151, Implementation.inc:1228-1267; tensor.comp:245-251):
 * dst[r][j] = row ids[r] (token id as raw bits) of the [vocab, dim] table w,
 * column j; 0 for ids at or past vocab.  w: F32, BF16, a packed GGUF
 * encoding, or S8 with `scales` = F32 [vocab] per-row scales.  rotation != 0
 * (ConvRot) -> QNN_E_NOT_SUPPORTED. */
int qnn_gather(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *ids, const qnn_weight *w, const qnn_weight *scales, int rows,
               int dim, int vocab, int rotation);

/* CachedAttention (Context.API.inc:142-146, Implementation.inc:1189-1226;
 * attention.comp): for query row r at absolute position position + r, softmax
 * attention over cache keys [start, position + r], start = end - window when
 * window > 0, of each head against its KV head (heads / kv_heads query heads
 * per KV head).  Scores are scaled by `scale` (0: 1/sqrt(dim)) and, when
 * softcap > 0, capped as softcap * tanh(score / softcap).  masked != 0 reads a
 * [query_rows][capacity] word mask after the cache; keys with a zero word are
 * skipped.  q, dst: [query_rows][heads][dim]; cache as GO_LLM_CACHE_WRITE. */
int qnn_cached_attention(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *q, qnn_tensor *cache, int query_rows, int capacity,
                         int heads, int kv_heads, int dim, int position, int window, float softcap, float scale,
                         int masked);

/* SampleToken (Context.API.inc:136-140, Implementation.inc:1137-1187;
 * tensor.comp:123-199): exact top-k (k = min(vocab, top_k), 1 at temperature
 * 0) of the logits after the repetition penalty (seen flag != 0: score * penalty
 * below zero, score / penalty above; flag 0xffffffff: token excluded), ranked
 * by score then lower id; then nucleus sampling with `uniform` in [0, 1).
 * dst[0] receives the token id as raw bits.  One launch for any vocabulary. */
int qnn_sample_token(qnn_ctx *ctx, qnn_tensor *dst, qnn_tensor *logits, qnn_tensor *seen, int vocab, int top_k,
                     float temperature, float top_p, float penalty, float uniform);

/* CheckFinite (Context.API.inc:158): a later qnn_download fails with
 * QNN_E_INVALID_OP if any checked value was NaN or infinite. */
int qnn_check_finite(qnn_ctx *ctx, qnn_tensor *t, int count);

/* ---------------------------------------------------------------------------
 * Routed experts on the device.  Replaces the host loop of TLLMMoE.forward
 * (src/models/QuickNN.Models.LLM.MoE.pas:376-448: route readback, per-expert
 * grouping, per-expert dispatches) for native-INT4 experts: all experts of a
 * layer are resident (registered once), routing and dispatch stay on the GPU
 * and only the routed experts' blocks are read.
 * ------------------------------------------------------------------------- */
/* gate/up: [inter, Int4RowBytes(hidden)]; down: [hidden, Int4RowBytes(inter)]; arrays of `experts`. */
int qnn_expert_set_create(qnn_ctx *ctx, const qnn_weight *gate, const qnn_weight *up, const qnn_weight *down,
                          int experts, int hidden, int inter, qnn_expert_set **out);
int qnn_expert_set_destroy(qnn_ctx *ctx, qnn_expert_set *set);
/* routes: output of GO_MOE_ROUTE ([rows*topk ids][rows*topk probabilities]).
 * dst[r] = sum over the token's routed experts in ascending id of
 *          p * down(silu(gate x_r) * (up x_r)).
 * One token (rows = 1) runs as a single launch outside graph capture
 * (QNN_FUSE_MOE=0 keeps the two-launch path); results are identical. */
int qnn_moe_experts(qnn_ctx *ctx, qnn_expert_set *set, qnn_tensor *dst, qnn_tensor *src, qnn_tensor *routes,
                    int rows, int topk);

/* ---------------------------------------------------------------------------
 * Diagnostics (no reference counterpart)
 * ------------------------------------------------------------------------- */
/* Writes the dequantized weight, fp32 [rows, cols], from the device-resident copy. */
int qnn_dequantize(qnn_ctx *ctx, qnn_tensor *dst, const qnn_weight *w, int rows, int cols);
/* HIP events on the context stream, for timing (slot < 64). */
int qnn_event_record(qnn_ctx *ctx, int slot);
int qnn_event_elapsed_ms(qnn_ctx *ctx, int slot_begin, int slot_end, float *ms);
/* Capture the ops recorded between begin and end into a HIP graph; replay it
 * with qnn_graph_launch.  All weights must already be resident. */
int qnn_graph_begin(qnn_ctx *ctx);
int qnn_graph_end(qnn_ctx *ctx, int *graph_id);
int qnn_graph_launch(qnn_ctx *ctx, int graph_id);
void *qnn_stream(qnn_ctx *ctx);

/* ---------------------------------------------------------------------------
 * Checkpoint files (host side; no context needed).  They turn safetensors and
 * GGUF checkpoints, and the INT4 cache built from them, into qnn_weight views
 * of the mapped bytes that the context's entry points take.
 * ------------------------------------------------------------------------- */
typedef struct qnn_tensor_files_s qnn_tensor_files; /* TSafeTensorFiles (SafeTensors.pas:207-222) */
typedef struct qnn_gguf_header_s qnn_gguf_header;   /* TGGUFHeader (GGUF.pas:26-34) */
typedef struct qnn_int4_cache_s qnn_int4_cache;     /* TLLMInt4Cache (LLM.Quantization.pas:13-28) */

/* TSafeTensor (SafeTensors.pas:149-180).  Pointers stay valid while the files are open. */
typedef struct {
  const char *name;       /* UTF-8, NUL-terminated */
  const void *data;       /* the mapped bytes */
  const int64_t *shape;   /* ndim dimensions, row-major (GGUF: reversed from ne[]) */
  uint64_t identity;      /* WeightIdentity: fresh per tensor per open, top bit set */
  int64_t data_offset;    /* DataOffset: absolute file offset */
  int64_t data_size;      /* DataSize: bytes */
  int32_t ndim;           /* Ndim */
  int32_t st_dtype;       /* DType: QNN_ST_* */
  int32_t dtype;          /* DType.ToDataType: QNN_DT_* (QNN_DT_UNDEF if none) */
  int32_t encoding;       /* Encoding: QNN_WE_* (packed GGUF blocks: not NATIVE) */
  int32_t file;           /* index of the file within the set */
  uint32_t storage_type;  /* GGML type of a GGUF tensor; 0xFFFFFFFF for safetensors */
} qnn_tensor_info;

/* TSafeTensorFile fields (SafeTensors.pas:184-197). */
typedef struct {
  const char *path;
  const char *architecture; /* GGUF general.architecture, else "" */
  const char *header_json;  /* HeaderJson: the raw safetensors header, "" for GGUF */
  const void *data;         /* Data: the mapping of the whole file */
  int64_t file_size, header_size, data_size, offset;
  int32_t is_gguf, tensor_count;
} qnn_tensor_file_info;

/* TSafeTensorFile.Open (SafeTensors.pas:522-690): a safetensors file, or a
 * GGUF file when its first four bytes are the GGUF magic (:480-520).  The
 * header is validated as the reference does (UTF-8, dtype sizes, contiguous
 * buffer with no gaps, overlaps or trailing bytes, unique names) and the file
 * is mapped read-only.  QNN_E_FORMAT on malformed files, QNN_E_IO if unreadable. */
int qnn_tensor_files_open(const char *path, qnn_tensor_files **out);
/* LoadSafeTensorShards (SafeTensors.pas:777-837): the shards named by
 * dir/index_file's weight_map, in order of first appearance, or dir/single_file
 * when there is no index. */
int qnn_tensor_files_open_shards(const char *dir, const char *index_file, const char *single_file,
                                 qnn_tensor_files **out);
int qnn_tensor_files_close(qnn_tensor_files *files);
int qnn_tensor_files_count(const qnn_tensor_files *files, int *count);
int qnn_tensor_files_file(const qnn_tensor_files *files, int file, qnn_tensor_file_info *out);
/* Tensors[index] of one file, in descriptor order. */
int qnn_tensor_files_tensor(const qnn_tensor_files *files, int file, int index, qnn_tensor_info *out);
/* GetTensor (SafeTensors.pas:900-912): the first file holding `name`; QNN_NOT_FOUND if none. */
int qnn_tensor_files_find(const qnn_tensor_files *files, const char *name, qnn_tensor_info *out);
/* GetLinearWeight(Name, UseMMAP = True) (SafeTensors.pas:874-898): packed GGUF
 * -> U8 view with its encoding and logical [N, K] shape; BF16 and F32 -> views
 * of the mapped data; F16 -> an F32 copy held until the files close.  A 1-D
 * tensor has shape1 = 1.  Missing tensor or other dtypes -> QNN_E_FORMAT. */
int qnn_tensor_files_linear_weight(qnn_tensor_files *files, const char *name, qnn_weight *out);

/* TGGUFHeader fields (GGUF.pas:26-34). */
typedef struct {
  uint32_t version, alignment;
  int64_t data_offset;
  int32_t vocabulary_size, tensor_count;
  const char *architecture;
  const char *metadata_json; /* the metadata object when requested, else "" */
} qnn_gguf_header_info;
/* TGGUFTensor (GGUF.pas:18-23). */
typedef struct {
  const char *name;
  const int64_t *shape; /* row-major, reversed from GGML ne[] */
  int64_t offset;       /* from the start of the data section */
  int64_t byte_size;
  int32_t ndim;
  uint32_t storage_type;
  int32_t encoding; /* GGUFEncoding(storage_type) */
} qnn_gguf_tensor;
/* TGGUFHeader.ReadFile (GGUF.pas:206-337): GGUF v2/v3 header and tensor table.
 * with_metadata != 0 collects the metadata as a JSON object (Metadata <> nil);
 * include_vocabulary = 0 skips the tokenizer vocabulary, merges, token types
 * and scores.  QNN_E_FORMAT on malformed headers, QNN_E_IO if unreadable. */
int qnn_gguf_read_file(const char *path, int with_metadata, int include_vocabulary, qnn_gguf_header **out);
int qnn_gguf_header_free(qnn_gguf_header *header);
int qnn_gguf_header_get(const qnn_gguf_header *header, qnn_gguf_header_info *out);
int qnn_gguf_header_tensor(const qnn_gguf_header *header, int index, qnn_gguf_tensor *out);

/* TLLMInt4Scope (LLM.Quantization.pas:11). */
#define QNN_IQ_EXPERTS 0
#define QNN_IQ_DENSE 1
/* TProc<Integer, Integer>: shards written so far and the shard count. */
typedef void (*qnn_progress_fn)(int done, int total, void *user);
/* TLLMInt4Cache.Create (LLM.Quantization.pas:79-125): opens the cache for
 * `sources` under directory/<format>-<fingerprint>, building it first when its
 * index is absent (:164-297: weight selection, QuantizeInt4 per matrix, shards
 * of 384 expert or 32 dense matrices, written as *.part and renamed, the index
 * last), then validates the index and every shard's metadata (:137-162).
 * A second builder of the same cache fails with QNN_E_IO while the first holds
 * its build.lock.  `sources` must stay open while the cache is built. */
int qnn_int4_cache_create(const qnn_tensor_files *sources, const char *directory, qnn_progress_fn progress,
                          void *user, int scope, qnn_int4_cache **out);
int qnn_int4_cache_destroy(qnn_int4_cache *cache);
/* Weight (LLM.Quantization.pas:299-317): U8 [rows, Int4RowBytes(columns)] of
 * the mapped shard; QNN_E_FORMAT if missing or of another shape. */
int qnn_int4_cache_weight(const qnn_int4_cache *cache, const char *name, int rows, int columns, qnn_weight *out);
/* MappedBytes (:319-325). */
int qnn_int4_cache_mapped_bytes(const qnn_int4_cache *cache, uint64_t *bytes);
/* Directory: NUL-terminated, valid while the cache is open. */
const char *qnn_int4_cache_directory(const qnn_int4_cache *cache);
/* SourceFingerprint (:70-73): 64 lowercase hex digits of SHA-256 plus NUL into out[65]. */
int qnn_int4_source_fingerprint(const qnn_tensor_files *sources, char *out);

/* ---------------------------------------------------------------------------
 * Host utilities
 * ------------------------------------------------------------------------- */
/* Int4RowBytes (src/core/QuickNN.Quantization.Int4.pas:25-33); -1 if invalid. */
int qnn_int4_row_bytes(int cols);
/* QuantizeInt4 (src/core/QuickNN.Quantization.Int4.pas:96-144): src F32 or BF16
 * [rows, cols] -> dst U8 [rows, Int4RowBytes(cols)].  Non-finite input -> QNN_E_ARGUMENT. */
int qnn_quantize_int4(const void *src, int dtype, int rows, int cols, uint8_t *dst);
/* GGML block encoder for synthetic weights (the reference ships no GGUF
 * quantizer): n elements (a multiple of the block size) -> blocks. */
int qnn_gguf_quantize(int encoding, const float *src, int64_t n, uint8_t *dst);

#ifdef __cplusplus
}
#endif
#endif
