// qnn_internal.h -- shared declarations of libqnn_hip.so (host + kernels).
#pragma once
#include <hip/hip_runtime.h>

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

// Integer tuning override from the environment (0 or unset: the default).
inline int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

// ---------------------------------------------------------------------------
// Device layouts
// ---------------------------------------------------------------------------
// Native INT4 tiled layout.  A packed INT4 matrix [N][G*20 B] (G = ceil(K/32)
// groups of fp32 scale + 16 nibble bytes) is stored as tiles of 64 rows, one
// row per lane of a wavefront:
//   nibble plane: 16 B at ((t*g4 + g)*64 + r)       -- group g of row r of tile t
//   scale plane:  16 B at ((t*(g4/4) + g/4)*64 + r)  -- scales of groups 4q..4q+3
// g4 = G rounded up to a multiple of 4.  Padding rows/groups carry nibble 8 and
// scale 0 (value 0).  The fused gate/up kernel reads two such matrices: lanes
// 0-31 stream 32 gate rows and lanes 32-63 the same 32 up rows.
struct I4Layout {
  int rows = 0, cols = 0, groups = 0, g4 = 0, tiles = 0;
  __host__ __device__ size_t nib_bytes() const { return size_t(tiles) * g4 * 64 * 16; }
  __host__ __device__ size_t scale_bytes() const { return size_t(tiles) * g4 * 64 * 4; }
  __host__ __device__ size_t bytes() const { return nib_bytes() + scale_bytes(); }
};

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
  WKind kind = WKind::Raw;
  void *dptr = nullptr;
  size_t bytes = 0;        // device bytes held
  size_t source_bytes = 0; // algorithmic (host) bytes
  int pins = 0;            // RetainWeight / graph references: never evicted
  int op_pins = 0;         // held during one call's acquisitions
  uint64_t last_use = 0;
  int raw_dtype = 0;       // Raw: dtype of the copied vector
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
  const void *nib = nullptr;   // tiled nibble plane (gate in I4_SWIGLU mode)
  const void *scl = nullptr;   // tiled scale plane
  const void *nib2 = nullptr;  // I4_SWIGLU: up matrix planes (same layout)
  const void *scl2 = nullptr;
  const float *x = nullptr;
  int x_stride = 0;  // floats between activation rows
  int x_vec4 = 0;    // x and x_stride allow 16-byte loads
  float *y = nullptr;
  int y_stride = 0;
  int k = 0, n = 0, m = 1;  // input features, valid output rows, tokens (<= 16)
  int tiles = 0, g4 = 0;    // wave tiles (64 output rows; 32 in I4_SWIGLU mode), groups/4*4
  int mode = I4_STORE;
  const float *prob = nullptr;  // I4_ACCUM: pointer to p
  float *partial = nullptr;     // split-K scratch
  unsigned *counters = nullptr;
  int xcd_local = 0;            // combine slices through the XCD's L2 (placement verified)
  int *err = nullptr;           // error word (bit 4: unexpected XCD placement)
};
bool xcd_probe(hipStream_t s);  // true when workgroup b runs on XCD b % 8
// Chooses the split-K slice and returns (partial floats, counters) needed.
void int4_plan(const I4Layout &l, int m, int *gs, int *slices);
size_t int4_partial_floats(const I4Layout &l, int m, int slices);
void int4_matvec_launch(const I4Launch &a, int gs, int slices, hipStream_t s);
void int4_repack_launch(const uint8_t *src, const I4Layout &l, void *dst, hipStream_t s);
I4Layout int4_layout(int rows, int cols);
void int4_dequant_launch(const I4Layout &l, const void *w, float *out, hipStream_t s);

void misc_fill(float *dst, int n, uint32_t bits, hipStream_t s);
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

// Device-side routed experts (qnn_moe.hip).  Every expert of a set is one
// contiguous tiled INT4 matrix per projection at base + e * stride.
constexpr int kMoEMaxExperts = 512;  // the route op's limit (moe.comp:13, 512-entry score array)
constexpr int kMoEMaxRoutes = 2048;  // rows * topk per call
struct MoELaunch {
  const uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
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
  int xcd_local = 0;
  int *err = nullptr;  // bit 8: invalid route ids
};
struct MoEPlanSizes {
  int slots = 0, mt = 1, gsw = 4, slices_gu = 1, slices_dn = 1;
  size_t partial_floats = 0, counters = 0;
};
MoEPlanSizes moe_plan(const MoELaunch &a);
void moe_launch(const MoELaunch &a, const MoEPlanSizes &p, hipStream_t s);

// Multi-row Q8_0 projection on fp16 MFMA (qnn_gemm.hip).
struct Q8GemmPlan {
  int m_pad = 0, k_pad = 0, ksteps = 0, mtiles = 0, ntiles = 0;
  size_t frag_bytes = 0, exp_bytes = 0;  // workspace: fp16 A fragments, per-row exponents
};
Q8GemmPlan q8_gemm_plan(int M, int K, int N);
void q8_gemm_launch(const Q8GemmPlan &p, const float *a, int M, int K, int N, const GGLayout &l, const void *w,
                    void *frag, int *ea, float *c, hipStream_t s);
void q8_rowexp_launch(const GGLayout &l, void *w, hipStream_t s);

// Persistent INT4 MLP layer stack (qnn_mlp.hip).
struct MlpLayerPtrs {
  const uint4 *gnib; const float *gscl;  // gate
  const uint4 *unib; const float *uscl;  // up
  const uint4 *dnib; const float *dscl;  // down
};
struct MlpArgs {
  const MlpLayerPtrs *w = nullptr;  // device array [layers]
  int layers = 0, hidden = 0, inter = 0;
  int g4_gu = 0, g4_d = 0, tiles_gu = 0, tiles_d = 0, slices_gu = 0, slices_d = 0;
  const float *x0 = nullptr;
  float *out = nullptr;
  float *hbuf = nullptr, *ybuf = nullptr;      // [2][inter], [2][hidden]
  float *part_gu = nullptr, *part_d = nullptr;  // [tiles][slices][64]
  unsigned *tick_gu = nullptr, *tick_d = nullptr;                 // stride kCounterStride
  unsigned long long *flag_gu = nullptr, *flag_d = nullptr;       // stride 8
  unsigned long long *epoch = nullptr;
  unsigned *exit_count = nullptr, *abort = nullptr;
  int *err = nullptr;
  unsigned spin_limit = 0;
};
int mlp_stack_grid(int gswu, int gswd, int want);
void mlp_stack_launch(const MlpArgs &a, int gswu, int gswd, int grid, hipStream_t s);

// GGUF (qnn_gguf.hip).
enum GGMode { GG_STORE = 0, GG_SWIGLU = 2 };
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
  float *partial = nullptr;
  unsigned *counters = nullptr;
  int xcd_local = 0;
  int *err = nullptr;
};
GGLayout gguf_layout(int enc, int rows, int cols);
void gguf_repack_launch(const uint8_t *src, const GGLayout &l, void *dst, hipStream_t s);
void gguf_dequant_launch(const GGLayout &l, const void *w, float *out, hipStream_t s);
void gguf_plan(const GGLayout &l, int tiles, int *bw, int *slices);
void gguf_matvec_launch(const GGArgs &a, int bw, int slices, hipStream_t s);

// Q8_0 GEMM (qnn_gemm.hip).
size_t q8_act_bytes(int m, int k);
void q8_act_quant_launch(const float *a, int m, int k, void *act, hipStream_t s);
void q8_gemm_launch(const GGLayout &l, const void *w, const void *act, int m, float *c, hipStream_t s);

}  // namespace qnn
