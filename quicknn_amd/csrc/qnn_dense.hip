// qnn_dense.hip -- projections over F32 / BF16 weights (row-major [out, in]).
//
// VectorLinear (Context.Implementation.inc:969-1001; ops GO_LLM_MATVEC /
// GO_LLM_MATVEC_BF16) and Linear with an F32 or BF16 weight
// (Implementation.inc:852-883, the gemm pipeline with the bf16 flag): the
// engine's router projection (LLM.MoE.pas:363-374) and the native-precision
// layers of the models.  bf16 weights widen to fp32 exactly (bits << 16);
// products and sums are fp32.
//
// * one row (dense_matvec_launch): one wave per output row; each lane reads
//   16-byte pieces of the row (4 fp32 or 8 bf16 weights) and the matching
//   activations, two pieces in flight per iteration, then a butterfly sum.
// * fused gate/up SwiGLU, one row (dense_swiglu_launch, op 66): as the
//   matvec, with the gate and up rows of an output read in the same pass.
// * several rows (dense_gemm_launch): a 256-thread workgroup computes a tile
//   of 64 outputs x 16 rows; 32-wide K slices of the weight tile and the
//   activation tile are staged in LDS (weights padded to 33 floats per row so
//   the 64 lanes of a wave read 64 different banks), and each thread
//   accumulates 4 rows of one output.
#include "qnn_internal.h"
#include "qnn_lanes.h"

namespace qnn {
namespace {

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// 16-byte piece i of a row as 4 (fp32) or 8 (bf16) floats, dotted with x.
template <bool BF16>
__device__ __forceinline__ float piece_dot(const uint4 w, const float *x) {
  if constexpr (BF16) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = fmaf(__uint_as_float(u[i] << 16), x[2 * i], s);
      s = fmaf(__uint_as_float(u[i] & 0xFFFF0000u), x[2 * i + 1], s);
    }
    return s;
  } else {
    float s = 0.0f;
    s = fmaf(__uint_as_float(w.x), x[0], s);
    s = fmaf(__uint_as_float(w.y), x[1], s);
    s = fmaf(__uint_as_float(w.z), x[2], s);
    s = fmaf(__uint_as_float(w.w), x[3], s);
    return s;
  }
}

// VEC: rows are whole 16-byte pieces and 16-byte aligned; otherwise one
// element per lane step.
template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void k_dense_matvec(const void *__restrict__ w, const float *__restrict__ x,
                                                      float *__restrict__ y, int n, int k) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;  // whole waves leave together
  float acc = 0.0f;
  if constexpr (VEC) {
    constexpr int E = BF16 ? 8 : 4;  // elements per 16-byte piece
    const int pieces = k / E;
    const uint4 *wr = reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(w) + size_t(row) * k * (BF16 ? 2 : 4));
    int p = lane;
    for (; p + 64 < pieces; p += 128) {  // two pieces in flight
      const uint4 a = wr[p], b = wr[p + 64];
      float xa[E], xb[E];
#pragma unroll
      for (int i = 0; i < E; i += 4) {
        const float4 va = *reinterpret_cast<const float4 *>(x + p * E + i);
        const float4 vb = *reinterpret_cast<const float4 *>(x + (p + 64) * E + i);
        xa[i] = va.x, xa[i + 1] = va.y, xa[i + 2] = va.z, xa[i + 3] = va.w;
        xb[i] = vb.x, xb[i + 1] = vb.y, xb[i + 2] = vb.z, xb[i + 3] = vb.w;
      }
      acc += piece_dot<BF16>(a, xa);
      acc += piece_dot<BF16>(b, xb);
    }
    if (p < pieces) {
      const uint4 a = wr[p];
      float xa[E];
#pragma unroll
      for (int i = 0; i < E; i += 4) {
        const float4 va = *reinterpret_cast<const float4 *>(x + p * E + i);
        xa[i] = va.x, xa[i + 1] = va.y, xa[i + 2] = va.z, xa[i + 3] = va.w;
      }
      acc += piece_dot<BF16>(a, xa);
    }
  } else {
    for (int j = lane; j < k; j += 64) {
      const float wv = BF16 ? bf16_to_f32(static_cast<const uint16_t *>(w)[size_t(row) * k + j])
                            : static_cast<const float *>(w)[size_t(row) * k + j];
      acc = fmaf(wv, x[j], acc);
    }
  }
  acc = dev::wave_sum_xor(acc);
  if (lane == 0) y[row] = acc;
}

// Weights j..j+7 of a row (16-byte aligned): one 16-byte piece of bf16, two
// of fp32.
template <bool BF16>
__device__ __forceinline__ void load8(const uint8_t *row, int j, float (&v)[8]) {
  if constexpr (BF16) {
    const uint4 p = *reinterpret_cast<const uint4 *>(row + size_t(j) * 2);
    const uint32_t u[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(u[i] << 16);
      v[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4 *>(row + size_t(j) * 4);
    const float4 b = *reinterpret_cast<const float4 *>(row + size_t(j) * 4 + 16);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
}
template <bool BF16>
__device__ __forceinline__ float weight_at(const void *w, size_t i) {
  return BF16 ? bf16_to_f32(static_cast<const uint16_t *>(w)[i]) : static_cast<const float *>(w)[i];
}

// Fused gate/up SwiGLU over F32 / BF16 weights, one row (TrySwiGLUVector's
// op 66, tensor.comp:38-48): h[r] = silu(Wg[r] . x) * (Wu[r] . x), the two
// rows read in one pass over x.  Gate and up may differ in type.  One wave
// per output row; VEC: rows are whole 8-element pieces, 16-byte aligned.
template <bool BG, bool BU, bool VEC>
__global__ __launch_bounds__(256) void k_dense_swiglu(const void *__restrict__ wg, const void *__restrict__ wu,
                                                      const float *__restrict__ x, float *__restrict__ y, int n,
                                                      int k) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;  // whole waves leave together
  float g = 0.0f, u = 0.0f;
  if constexpr (VEC) {
    const uint8_t *rg = static_cast<const uint8_t *>(wg) + size_t(row) * k * (BG ? 2 : 4);
    const uint8_t *ru = static_cast<const uint8_t *>(wu) + size_t(row) * k * (BU ? 2 : 4);
    for (int j = lane * 8; j < k; j += 512) {
      float a[8], b[8], xv[8];
      load8<BG>(rg, j, a);
      load8<BU>(ru, j, b);
      const float4 x0 = *reinterpret_cast<const float4 *>(x + j), x1 = *reinterpret_cast<const float4 *>(x + j + 4);
      xv[0] = x0.x, xv[1] = x0.y, xv[2] = x0.z, xv[3] = x0.w, xv[4] = x1.x, xv[5] = x1.y, xv[6] = x1.z, xv[7] = x1.w;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        g = fmaf(a[i], xv[i], g);
        u = fmaf(b[i], xv[i], u);
      }
    }
  } else {
    for (int j = lane; j < k; j += 64) {
      const float xv = x[j];
      g = fmaf(weight_at<BG>(wg, size_t(row) * k + j), xv, g);
      u = fmaf(weight_at<BU>(wu, size_t(row) * k + j), xv, u);
    }
  }
  g = dev::wave_sum_xor(g);
  u = dev::wave_sum_xor(u);
  if (lane == 0) {
    const float sg = g >= 20.0f ? g : (g <= -20.0f ? 0.0f : g / (1.0f + expf(-g)));  // tensor.comp:22
    y[row] = sg * u;
  }
}

constexpr int kTN = 64, kTM = 16, kTK = 32;

template <bool BF16>
__global__ __launch_bounds__(256) void k_dense_gemm(const void *__restrict__ w, const float *__restrict__ x,
                                                    float *__restrict__ y, int m, int n, int k) {
  __shared__ float ws[kTN][kTK + 1];
  __shared__ float xs[kTM][kTK];
  const int t = threadIdx.x;
  const int n0 = blockIdx.x * kTN, m0 = blockIdx.y * kTM;
  const int nl = t & 63, mg = t >> 6;  // output n0 + nl, rows m0 + 4*mg .. +3
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < k; k0 += kTK) {
#pragma unroll
    for (int i = 0; i < kTN * kTK / 256; ++i) {  // weight tile: 8 elements per thread
      const int e = i * 256 + t, r = e / kTK, c = e % kTK;
      const int gn = n0 + r, gk = k0 + c;
      float v = 0.0f;
      if (gn < n && gk < k)
        v = BF16 ? bf16_to_f32(static_cast<const uint16_t *>(w)[size_t(gn) * k + gk])
                 : static_cast<const float *>(w)[size_t(gn) * k + gk];
      ws[r][c] = v;
    }
#pragma unroll
    for (int i = 0; i < kTM * kTK / 256; ++i) {  // activation tile: 2 elements per thread
      const int e = i * 256 + t, r = e / kTK, c = e % kTK;
      const int gm = m0 + r, gk = k0 + c;
      xs[r][c] = gm < m && gk < k ? x[size_t(gm) * k + gk] : 0.0f;
    }
    __syncthreads();
#pragma unroll 8
    for (int c = 0; c < kTK; ++c) {
      const float wv = ws[nl][c];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(wv, xs[4 * mg + i][c], acc[i]);
    }
    __syncthreads();
  }
  const int gn = n0 + nl;
  if (gn < n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int gm = m0 + 4 * mg + i;
      if (gm < m) y[size_t(gm) * n + gn] = acc[i];
    }
  }
}

}  // namespace

void dense_matvec_launch(const void *w, int bf16, const float *x, float *y, int n, int k, hipStream_t s) {
  const int es = bf16 ? 2 : 4;
  const bool vec = (size_t(k) * es) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(x) % 16 == 0;
  const dim3 grid((n + 3) / 4), block(256);
  if (bf16) {
    if (vec) hipLaunchKernelGGL((k_dense_matvec<true, true>), grid, block, 0, s, w, x, y, n, k);
    else hipLaunchKernelGGL((k_dense_matvec<true, false>), grid, block, 0, s, w, x, y, n, k);
  } else {
    if (vec) hipLaunchKernelGGL((k_dense_matvec<false, true>), grid, block, 0, s, w, x, y, n, k);
    else hipLaunchKernelGGL((k_dense_matvec<false, false>), grid, block, 0, s, w, x, y, n, k);
  }
  hip_check(hipGetLastError(), "dense matvec launch");
}

void dense_swiglu_launch(const void *wg, int bg, const void *wu, int bu, const float *x, float *y, int n, int k,
                         hipStream_t s) {
  const bool vec = k % 8 == 0 && reinterpret_cast<uintptr_t>(wg) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(wu) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  const dim3 grid((n + 3) / 4), block(256);
#define QNN_SWIGLU_CASE(G, U)                                                                     \
  if (bool(bg) == G && bool(bu) == U) {                                                          \
    if (vec) hipLaunchKernelGGL((k_dense_swiglu<G, U, true>), grid, block, 0, s, wg, wu, x, y, n, k); \
    else hipLaunchKernelGGL((k_dense_swiglu<G, U, false>), grid, block, 0, s, wg, wu, x, y, n, k);    \
  }
  QNN_SWIGLU_CASE(false, false)
  QNN_SWIGLU_CASE(false, true)
  QNN_SWIGLU_CASE(true, false)
  QNN_SWIGLU_CASE(true, true)
#undef QNN_SWIGLU_CASE
  hip_check(hipGetLastError(), "dense swiglu launch");
}

void dense_gemm_launch(const void *w, int bf16, const float *x, float *y, int m, int n, int k, hipStream_t s) {
  const dim3 grid((n + kTN - 1) / kTN, (m + kTM - 1) / kTM), block(256);
  if (bf16) hipLaunchKernelGGL(k_dense_gemm<true>, grid, block, 0, s, w, x, y, m, n, k);
  else hipLaunchKernelGGL(k_dense_gemm<false>, grid, block, 0, s, w, x, y, m, n, k);
  hip_check(hipGetLastError(), "dense gemm launch");
}

}  // namespace qnn
