// qnn_internal.h -- shared declarations of libqnn_hip.so (host + kernels).
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <list>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/qnn_hip.h"

namespace qnn {

// Error carrying one of the QNN_E_* codes; converted to a status at the C ABI.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] inline void fail(int code, const std::string &msg) { throw Error(code, msg); }
inline void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) fail(QNN_E_INVALID_OP, std::string(what) + ": " + hipGetErrorString(e));
}
// a + b*c with the product rounded before the sum (never fused into an fma):
// the accumulate of moe.comp:70 / :126 as the reference's CPU path computes it.
__host__ __device__ inline float add_mul_nofma(float a, float b, float c) {
#pragma clang fp contract(off)
  return a + b * c;
}

// Tuning switches: QNN_* environment variables read into one snapshot when a
// context is created (and by qnn_reload_tuning), never per launch.  A value of
// 0 in the planners' fields means "the planner's own choice".
struct Tuning {
  int group_linear = 1;      // QNN_GROUP_LINEAR: grouped one-row GGUF Linear launches
  int fuse_mlp = 1;          // QNN_FUSE_MLP: recorded INT4 SwiGLU + down as one launch
  int fuse_moe = 1;          // QNN_FUSE_MOE: one-token routed experts (and route) as one launch
  int q8_gemm_min_rows = 4;  // QNN_Q8_GEMM_MIN_ROWS: rows from which Q8_0 Linear takes the GEMM
  int gemm_h16 = 128;        // QNN_GEMM_H16: rows from which Q8_0 Linear runs over a pre-expanded fp16 copy (0: never)
  int gguf_gemm_rows = 12;   // QNN_GGUF_GEMM_ROWS: the same for the other GGUF encodings (0: never)
  int gemm_max_rows = 0;     // QNN_GEMM_MAX_ROWS: rows per GEMM launch, at most (0: the 4 GiB fragment limit)
  int attn_wgs = 512;        // QNN_ATTN_WGS: cached-attention workgroup target
  int attn_min_chunk = 64;   // QNN_ATTN_MIN_CHUNK: keys per chunk, at least
  int attn_dma = 1;          // QNN_ATTN_DMA: 64-key chunks at dim 128 streamed into LDS
  int gemm_nw = 0;           // QNN_GEMM_NW: waves per Q8_0 GEMM workgroup (4 or 8)
  int gemm_mb = 0;           // QNN_GEMM_MB: 32-row blocks per GEMM wave (1 or 2)
  int gg_bw = 0;             // QNN_GG_BW: GGUF units per wave (1 or 2)
  int gg_mt = 1;             // QNN_GG_MT: GGUF Linear below the GEMM, up to 8 rows per pass (0: one per row)
  int i4_mfma = 1;           // QNN_I4_MFMA: multi-token INT4 dot on the int8 matrix cores
  int i4_lanes = 0;          // QNN_I4_LANES: lanes per INT4 row at upload (1..16)
  int i4_tpw = 1;            // QNN_I4_TPW: INT4 tiles per workgroup (1, 2, 4)
  int i4_target_waves = 0;   // QNN_I4_TARGET_WAVES: wave target of the INT4 planner
  int i4_sps = 0;            // QNN_I4_SPS: INT4 steps per wave
  int i4_wide = 1;           // QNN_I4_WIDE: one-token 8/16-wave workgroups
  int moe_mt = 0;            // QNN_MOE_MT: tokens per pass of the multi-token MoE kernels
  int moe_sps = 0;           // QNN_MOE_SPS: MoE steps per wave
};
const Tuning &tuning();
void reload_tuning();

// ---------------------------------------------------------------------------
// Device layouts
// ---------------------------------------------------------------------------
// Native INT4 device layout (qnn_int4_dev.h).  A packed INT4 matrix
// [N][G*20 B] (G = ceil(K/32) groups of fp32 scale + 16 nibble bytes) is held
// as 64-lane blocks of R = 64/L rows, L lanes per row; lane l = r*L + j of
// block b carries groups j, j+L, ... of row b*R + r, step s at
//   nibbles: 16 B at ((b*S + s)*64 + l),   scales: 4 B at ((b*S + s)*64 + l)
// with S = ceil(G / L) steps.  Padding rows/groups hold scale 0 and nibble 8.
struct I4Layout {
  int rows = 0, cols = 0, groups = 0;
  int lanes = 1;   // L: lanes per row (power of two <= 16)
  int rpb = 64;    // R = 64 / L rows per block
  int steps = 0;   // S
  int blocks = 0;  // ceil(rows / R)
  __host__ __device__ int quads() const { return (steps + 3) / 4; }  // scale pieces: 4 steps each
  __host__ __device__ size_t nib_bytes() const { return size_t(blocks) * steps * 64 * 16; }
  __host__ __device__ size_t scale_bytes() const { return size_t(blocks) * quads() * 64 * 16; }
  // Float index of the scale of step s, lane l, block b.
  __host__ __device__ size_t scale_at(int b, int s, int l) const {
    return ((size_t(b) * quads() + (s >> 2)) * 64 + l) * 4 + (s & 3);
  }
  __host__ __device__ size_t bytes() const { return nib_bytes() + scale_bytes(); }
};

// fp16 operands of the GEMMs: exponent e with |v| * 2^-e in (2^13, 2^14] (0
// for zero or non-finite v), and two round-to-nearest-even fp16 in a dword.
__device__ __forceinline__ int range_exp(float amax) {
  if (!(amax > 0.0f) || !isfinite(amax)) return 0;
  int ex;
  (void)frexpf(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
  return ex - 14;
}
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  const _Float16 x = _Float16(a), y = _Float16(b);
  uint16_t u, v;
  __builtin_memcpy(&u, &x, 2);
  __builtin_memcpy(&v, &y, 2);
  return uint32_t(u) | (uint32_t(v) << 16);
}

// GGUF tiled layout (qnn_gguf.hip): tiles of 64 rows, 256-element units,
// a 16-byte-aligned main plane plus up to two small side planes.
struct GGLayout {
  int enc = 0, rows = 0, cols = 0, tiles = 0, units = 0;
  int main_chunks = 0, side1_bytes = 0, side2_bytes = 0, unit_bytes = 0, src_row_bytes = 0;
  size_t side1_off = 0, side2_off = 0, total = 0;
  size_t rowexp_off = 0;  // Q8_0: int per row, the GEMM's fp16 range exponent (qnn_gemm.hip)
  size_t bytes() const { return total; }
};

enum class WKind { Int4, Gguf, Raw };

struct WeightEntry {
  std::string key;
  uint64_t identity = 0;   // WeightIdentity of the source block (reported on eviction)
  WKind kind = WKind::Raw;
  void *dptr = nullptr;
  size_t bytes = 0;        // device bytes held
  size_t source_bytes = 0; // algorithmic (host) bytes
  int pins = 0;            // RetainWeight / graph references: never evicted
  int op_pins = 0;         // held during one call's acquisitions
  uint64_t last_use = 0;
  int raw_dtype = 0;       // Raw: dtype of the copied vector
  hipEvent_t ready = nullptr;  // written by an asynchronous prefetch: the compute stream waits for it first
  bool derived = false;        // made on the device from another entry (the fp16 copy of a Q8_0 weight):
                               // its eviction is not reported through OnWeightEvicted
  I4Layout i4;
  GGLayout gg;
};

struct Tensor {
  float *ptr = nullptr;
  int count = 0;
  size_t capacity = 0;
  bool live = false;
};

// ---------------------------------------------------------------------------
// Kernel launchers (device code in qnn_int4.hip / qnn_misc.hip / ...)
// ---------------------------------------------------------------------------
enum I4Mode { I4_STORE = 0, I4_ACCUM = 1, I4_SWIGLU = 2 };

// Split-K tickets sit 256 bytes apart: atomics on one cache line serialise in
// a single L2 channel (about 16 ns each), so neighbouring tiles must not share.
constexpr int kCounterStride = 64;

struct I4Launch {
  I4Layout l;                  // layout of the (gate) matrix
  const void *nib = nullptr;   // nibble plane (gate in I4_SWIGLU mode)
  const void *scl = nullptr;   // scale plane
  const void *nib2 = nullptr;  // I4_SWIGLU: up matrix planes (same layout)
  const void *scl2 = nullptr;
  const float *x = nullptr;  // rows of k floats (k % 4 == 0, 16-byte aligned), x_stride apart
  int x_stride = 0;
  float *y = nullptr;
  int y_stride = 0;
  int k = 0, n = 0, m = 1;  // input features, valid output rows, tokens
  int tiles = 0;            // wave tiles: blocks (I4_SWIGLU: 2 per block, 32 lanes of gate + 32 of up)
  int steps_per_slice = 0;  // steps per wave (a workgroup slice is 4/T times that)
  int mode = I4_STORE;
  const float *prob = nullptr;  // I4_ACCUM: pointer to p
  float *g_out = nullptr;       // I4_SWIGLU, optional: the gate and up sums too (y_stride apart)
  float *u_out = nullptr;
  float *partial = nullptr;     // split-K scratch
  unsigned *counters = nullptr;
  int *err = nullptr;           // error word
};
struct I4Plan {
  int mt = 1, gsw = 1, slices = 1, grid = 0, steps_per_slice = 1, tiles_per_wg = 1;
  int wg_waves = 4;           // 8 or 16: one workgroup takes what 2 or 4 four-wave slices would
  size_t lds = 0;             // dynamic LDS bytes
  size_t partial_floats = 0;  // split-K scratch
  size_t counters = 0;
};
// Launch geometry for m tokens (at most 16 per launch) in the given mode.
// wide: the plan may take 8- or 16-wave workgroups (k_int4_matvec only; the
// fused kernels build their items from the four-wave plan).
I4Plan int4_plan(const I4Layout &l, int m, int mode, bool wide = false);
void int4_matvec_launch(const I4Launch &a, const I4Plan &p, hipStream_t s);
void int4_repack_launch(const uint8_t *src, const I4Layout &l, void *dst, hipStream_t s);
// one_lane: one lane per row whatever QNN_I4_LANES says (the MoE expert kernels assume it).
I4Layout int4_layout(int rows, int cols, bool one_lane = false);
void int4_dequant_launch(const I4Layout &l, const void *w, float *out, hipStream_t s);

void misc_fill(float *dst, int n, uint32_t bits, hipStream_t s);
void misc_stream_read(const void *src, size_t bytes, uint32_t *out, hipStream_t s);  // diagnostic HBM stream
void misc_add(float *dst, const float *a, int n, int cols, int dst_stride, float alpha, int dst_off, int src_off,
              hipStream_t s);
void misc_glu(float *dst, const float *a, const float *b, int n, int inter, int interleaved, int gelu,
              hipStream_t s);
void misc_finite(const float *a, int n, int *flag, hipStream_t s);
void misc_norm(float *dst, const float *a, const void *gamma, int gamma_bf16, const void *beta, int beta_bf16,
               int rows, int dim, int flags, int src_off, int unit_gamma, float eps, hipStream_t s);
void misc_moe_route(float *routes, const float *logits, int rows, int experts, int k, int normalize,
                    hipStream_t s);
void misc_moe_gather(float *dst, const float *src, size_t src_n, const float *indices, int n, int hidden, int topk,
                     int offset, int *err, hipStream_t s);
void misc_moe_scatter(float *dst, size_t dst_n, const float *y, const float *indices, const float *routes,
                      size_t routes_n, int n, int hidden, int topk, int offset, int route_index, int single_row,
                      int prob_base, int *err, hipStream_t s);
void misc_bias_add(float *dst, const void *bias, int bias_bf16, int rows, int cols, hipStream_t s);
void misc_pad_rows(float *dst, const float *src, int rows, int cols, int cols_pad, hipStream_t s);

// Decode-layer ops (qnn_decode.hip).
void decode_rope(float *dst, const float *src, int n, int heads, int dim, int position, float theta, hipStream_t s);
void decode_cache_write(float *cache, const float *k, const float *v, int n, int kv_heads, int dim, int cap,
                        int position, hipStream_t s);
void decode_seen(float *flags, const float *ids, int n, int vocab, hipStream_t s);
void decode_scale(float *dst, const float *src, int n, float a, float b, hipStream_t s);
// kind: 0 F32, 1 BF16, 2 int8 with per-row F32 scales.
void decode_gather(float *dst, const float *ids, const void *w, int kind, const float *scales, int rows, int dim,
                   int vocab, hipStream_t s);
void gguf_gather_launch(const GGLayout &l, const void *w, const float *ids, float *out, int rows, int vocab,
                        hipStream_t s);
void decode_softcap(float *dst, const float *src, int n, float cap, hipStream_t s);
// Cached attention: query heads per workgroup (gb), key chunks (splits) and
// the chunk partials' workspace in floats (0 when one chunk covers the keys).
struct AttnPlan {
  int gb = 1, splits = 1, chunk = 64;
  size_t part_floats = 0;
};
AttnPlan attn_plan(int rows, int heads, int kv_heads, int dim, int position, int window);
void attn_launch(const float *q, const float *cache, float *out, float *ws, const AttnPlan &p, int rows, int cap,
                 int heads, int kv_heads, int dim, int position, int window, float softcap, float scale, int masked,
                 hipStream_t s);
// Token sampling: tiles of 4096 tokens per level; the candidates of every
// level take sample_workspace_floats words.
size_t sample_workspace_floats(int vocab, int k);
void sample_launch(float *dst, const float *logits, const float *seen, float *ws, unsigned *counter, int vocab, int k,
                   float temperature, float top_p, float penalty, float uniform, hipStream_t s);

// Device-side routed experts (qnn_moe.hip).  Every expert of a set is one
// contiguous tiled INT4 matrix per projection at base + e * stride.
constexpr int kMoEMaxExperts = 512;  // the route op's limit (moe.comp:13, 512-entry score array)
constexpr int kMoEMaxRoutes = 2048;  // rows * topk per call
// One decode MLP in a single launch (qnn_mlp.hip): gate/up items
// of the I4_SWIGLU plan and down items of the I4_STORE plan.
struct MlpLaunch {
  I4Layout lg, ld;  // gate/up layout (both matrices), down layout; one lane per row
  const void *gnib = nullptr, *gscl = nullptr, *unib = nullptr, *uscl = nullptr, *dnib = nullptr, *dscl = nullptr;
  const float *x = nullptr;  // hidden floats
  float *h = nullptr;        // inter floats (written, device-coherent)
  float *y = nullptr;        // hidden floats
  int hidden = 0, inter = 0;
  int sps_gu = 0, slices_gu = 0;             // I4_SWIGLU plan of the pair
  int sps_dn = 0, slices_dn = 0, grid_dn = 0;  // I4_STORE plan of the down matrix (its per-op grid)
  float *partial_gu = nullptr, *partial_dn = nullptr;
  unsigned *counters_gu = nullptr, *counters_dn = nullptr;
  unsigned *flags = nullptr;  // per 64-row block of h, 256 B apart: epoch of the launch that completed it
  unsigned epoch = 0;         // this launch's number (never 0)
  int *err = nullptr;         // bit 2: a wait for h timed out
};
size_t mlp_lds_bytes(int gg, int gd);
int mlp_capacity(int gg, int gd, int device);  // co-resident workgroups (0: variant not built)
bool mlp_launch(const MlpLaunch &a, int gg, int gd, int grid, hipStream_t s);  // false: not launched

// Phase timestamps of the fused MLP kernels (trace builds only): copies up to
// `bytes` of [workgroup][16] u64 and clears them; words copied, -2 when the
// library is not a trace build, -1 on a HIP error.
int mlp_phase_read(void *dst, size_t bytes);
int moe_phase_read(void *dst, size_t bytes);   // the one-token MoE kernel's, likewise
int attn_phase_read(void *dst, size_t bytes);  // the LDS-streamed attention kernel's, likewise

struct MoELaunch {
  const uint8_t *gate_up = nullptr;  // expert e: gate at gate_up + 2e*gu_stride, its up matrix gu_stride after it
  const uint8_t *down = nullptr;     // expert e: down + e*dn_stride
  size_t gu_stride = 0, dn_stride = 0;  // bytes per expert matrix
  I4Layout gu, dn;                      // gate/up [inter, hidden]; down [hidden, inter]
  int experts = 0, hidden = 0, inter = 0, topk = 0, rows = 0;
  const float *x = nullptr;       // [rows][hidden]
  const float *routes = nullptr;  // [rows*topk ids as u32][rows*topk probabilities]
  float *out = nullptr;           // [rows][hidden]
  float *h = nullptr;             // workspace [rows*topk][inter]
  float *y = nullptr;             // workspace [rows*topk][hidden]
  float *partial = nullptr;
  unsigned *counters = nullptr;
  int *plan = nullptr;  // multi-token launches: slot plans written by k_moe_plan (plan_words words)
  int *err = nullptr;   // bit 8: invalid route ids; bit 2: a fused-launch wait for h timed out
  // single-launch decode path (one token) only:
  float *partial_dn = nullptr;
  unsigned *counters_dn = nullptr;
  unsigned *flags = nullptr;  // per (slot, 64-row block of h), 256 B apart: epoch of the launch that completed it
  unsigned epoch = 0;
  // computing the routes in the launch (moe_decode_launch with route_j > 0):
  const float *logits = nullptr;  // [experts] router logits of the token
  float *routes_out = nullptr;    // the route tensor, written as GO_MOE_ROUTE would
  int normalize = 0;
};
struct MoEPlanSizes {
  int slots = 0, mt = 1, gsw = 4, slices_gu = 1, slices_dn = 1, sps_gu = 1, sps_dn = 1;
  size_t lds_gu = 0, lds_dn = 0;  // dynamic LDS per launch
  size_t partial_floats = 0, counters = 0;
  size_t plan_words = 0;  // slot plans of the multi-token launches (k_moe_plan)
};
// One-token MoE as a single launch: sizes of its workspace and grid.
struct MoEDecodePlan {
  bool ok = false;  // shape and plan allow the single launch
  int grid = 0, grid_dn = 0, units_gu = 0, bpad_dn = 0;
  size_t partial_gu = 0, partial_dn = 0, counters_gu = 0, counters_dn = 0, flag_bytes = 0;  // floats / words / bytes
};
MoEDecodePlan moe_decode_plan(const MoELaunch &a, const MoEPlanSizes &p);
int moe_route_j(int experts);  // route-computing variant for this expert count (0: none)
int moe_decode_capacity(const MoEPlanSizes &p, int route_j, int device);  // co-resident workgroups (0: not built)
bool moe_decode_launch(const MoELaunch &a, const MoEPlanSizes &p, const MoEDecodePlan &d, int route_j, hipStream_t s);
MoEPlanSizes moe_plan(const MoELaunch &a);
void moe_launch(const MoELaunch &a, const MoEPlanSizes &p, hipStream_t s);

// Multi-row Q8_0 projection on fp16 MFMA (qnn_gemm.hip).
struct Q8GemmPlan {
  int mb = 1;  // 32-row blocks of C per wave
  int nw = 4;  // waves per workgroup (workgroup tile 32 * mb * nw rows)
  int m_pad = 0, k_pad = 0, ksteps = 0, mtiles = 0, ntiles = 0;
  size_t frag_bytes = 0, exp_bytes = 0;  // workspace: fp16 A fragments, per-row exponents
};
Q8GemmPlan q8_gemm_plan(int M, int K, int N);
void q8_gemm_launch(const Q8GemmPlan &p, const float *a, int M, int K, int N, const GGLayout &l, const void *w,
                    void *frag, int *ea, float *c, hipStream_t s);
void q8_rowexp_launch(const GGLayout &l, void *w, hipStream_t s);
// The same product over a pre-expanded fp16 copy of the weight (qnn_gemm.hip,
// k_h16_gemm): q8_h16_bytes of device memory per weight, made once by
// q8_expand_h16_launch; the results equal q8_gemm_launch's bit for bit.
// `ew` is the weight's row exponents (a Q8_0 weight's own, at rowexp_off).
size_t q8_h16_bytes(int rows, int cols);
void q8_expand_h16_launch(const GGLayout &l, const void *w, void *out, hipStream_t s);
Q8GemmPlan q8_h16_plan(int M, int K, int N);
// ksplit > 1 (h16_ksplit: small grids) splits K over that many workgroups per
// tile, their partial products in `part` (ksplit * M * N floats, N % 4 == 0),
// summed in slice order by a second launch; ksplit 1 writes C directly.
int h16_ksplit(const Q8GemmPlan &p, int N);
void q8_h16_gemm_launch(const Q8GemmPlan &p, const float *a, int M, int K, int N, const int *ew, const void *w16,
                        void *frag, int *ea, float *c, hipStream_t s, int ksplit = 1, float *part = nullptr);
// The fp16 copy of a weight of any other GGUF encoding (qnn_gguf.hip): its
// row exponents (range_exp of the row's largest |value|, one int per row of
// the copy's q8_h16_bytes rows), then the values RNE(v * 2^-e) in
// k_h16_gemm's fragment order.
void gguf_rowexp_launch(const GGLayout &l, const void *w, int *ew, int rows_pad, hipStream_t s);
void gguf_expand_h16_launch(const GGLayout &l, const void *w, const int *ew, void *out, hipStream_t s);
// Multi-row Q8_0 projection with activations quantised per 32-element block to
// int8, on the int8 matrix cores (qnn_gemm_i8.hip).  K % 32 == 0.
size_t q8_i8_workspace(int M, int K);
void q8_gemm_i8_launch(const float *a, int M, int K, int N, const GGLayout &l, const void *w, void *ws, float *c,
                       hipStream_t s);


// Fixed device scratch of the no-allocation INT4 projection (qnn_noalloc.hip):
// [split-K partial sums: 7 MiB][arrival tickets: 1 MiB], one copy per GPU.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
constexpr size_t kNoAllocCounterBytes = size_t(1) << 20;
constexpr size_t kNoAllocPartialBytes = kNoAllocScratchBytes - kNoAllocCounterBytes;
void noalloc_scratch_init(int device);  // with `device` current: resolves and keeps its copy's address
void *noalloc_scratch(int device);      // that address, or null if set-up failed

// F32 / BF16 weights, row-major [n, k] (qnn_dense.hip): y = W x for one row,
// Y[m, n] = X[m, k] W^T for several.
void dense_matvec_launch(const void *w, int bf16, const float *x, float *y, int n, int k, hipStream_t s);
void dense_gemm_launch(const void *w, int bf16, const float *x, float *y, int m, int n, int k, hipStream_t s);
// h = silu(Wg x) * (Wu x) for one row; gate and up each F32 (0) or BF16 (1).
void dense_swiglu_launch(const void *wg, int bg, const void *wu, int bu, const float *x, float *y, int n, int k,
                         hipStream_t s);

// GGUF (qnn_gguf.hip).
enum GGMode { GG_STORE = 0, GG_SWIGLU = 2, GG_GEGLU = 3 };
struct GGArgs {
  GGLayout l;
  const void *w = nullptr;   // tiled weight (gate in pair modes)
  const void *w2 = nullptr;  // pair modes: up weight (same layout)
  const float *x = nullptr;
  int x_vec4 = 0;
  float *y = nullptr;
  int n = 0;       // valid output rows
  int tiles = 0;   // wave tiles (64 rows; 32 in pair modes)
  int mode = GG_STORE;
  float *g_out = nullptr;  // pair modes, optional: the gate and up sums too
  float *u_out = nullptr;
  float *partial = nullptr;
  unsigned *counters = nullptr;
  int *err = nullptr;
};
GGLayout gguf_layout(int enc, int rows, int cols);
void gguf_repack_launch(const uint8_t *src, const GGLayout &l, void *dst, hipStream_t s);
void gguf_dequant_launch(const GGLayout &l, const void *w, float *out, hipStream_t s);
void gguf_plan(const GGLayout &l, int tiles, int *bw, int *slices);
void gguf_matvec_launch(const GGArgs &a, int bw, int slices, hipStream_t s);
// 2 to kGGMaxTokens tokens (rows of a.x, a.x row stride a.l.cols, a.y row
// stride a.n) in one pass over the weights, one unit per wave (qnn_gguf.hip).
// Needs kGGMaxTokens partial sums per split-K slot.
constexpr int kGGMaxTokens = 8;
void gguf_matvec_mt_launch(const GGArgs &a, int slices, int ntok, hipStream_t s);
// Up to kGGMaxGroup matvecs of one encoding and plan width in one launch:
// member i owns workgroups [start[i], start[i+1]) (multiples of 8, so each
// member keeps its XCD-aware tile map).
constexpr int kGGMaxGroup = 4;
struct GGGroup {
  GGArgs m[kGGMaxGroup];
  int slices[kGGMaxGroup] = {};
  int start[kGGMaxGroup + 1] = {};
  int count = 0;
};
void gguf_group_launch(const GGGroup &g, int bw, hipStream_t s);

}  // namespace qnn
