// qnn_gemm_i8.hip -- multi-row Q8_0 projection with int8 activations on the
// int8 matrix cores (the benchmark's prefill GEMM: activations quantised per
// 32-element block to int8, weights Q8_0 as stored).
//
//   K7  q8 activation quantiser: per row m and 32-element block b,
//         d = max|x| / 127,  id = d != 0 ? 1 / d : 0,  q = roundf(x * id)
//       (the public GGML reference rule for Q8_0 blocks, with d kept in fp32).
//   K8  C[m][n] = sum over b, in ascending order, of
//         acc = fma(float(S_b[m][n]), dx[m][b] * dw[n][b], acc),
//       S_b = the exact int32 dot of block b's int8 activations and int8
//       weights (one v_mfma_i32_32x32x32_i8 per 32 x 32 tile and block),
//       dw = the block's fp16 scale (exact in fp32).
// Every step is exact or one IEEE rounding in a fixed order, so the result is
// reproducible bit for bit by a CPU restatement.  It differs from the
// reference's fp32-activation product (gemm.comp, GGUF.Quantization.pas:
// 247-258) by the activation quantisation (about 5e-3 normwise for N(0, 1)
// activations); Linear (qnn_gemm.hip) keeps fp32-level agreement instead.
//
// Each block needs its own pair of scales, so the epilogue costs three VALU
// operations per output per block (convert, scale product, fma): at the cfg5
// shape 512 x 12288 x 96 blocks that is 1.8 G lane-operations, against 7.7 us
// of int8 MFMA work -- this kernel is bound by the VALU, not the matrix cores.
//
// Tiling: a 256-thread workgroup computes 64 rows x 128 columns; wave w takes
// rows 32 * (w & 1) and columns 64 * (w >> 1) as two 32 x 32 MFMA tiles.
// Activations come pre-arranged in MFMA fragment order (16 bytes per lane and
// block, one coalesced 1 KiB load per 32 rows); weight fragments are read
// straight from the tiled Q8_0 layout (lane l: row l % 32 of the tile, the
// 16 quants of half l / 32 of the block: 512 contiguous bytes per half).  All
// M-tiles of an N-tile share blockIdx % 8, so they run on one XCD and the
// weights come from HBM once.
#include "qnn_internal.h"

namespace qnn {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(uint32_t(min(bytes, size_t(0xFFFFFFFFu)))),
                                           0x00020000);
}
constexpr uint32_t kOutside = 0xFFFFFFF0u;  // a buffer offset past the end: loads return 0

__device__ __forceinline__ float half_to_f(uint32_t h) {
  const uint16_t b = uint16_t(h);
  _Float16 f;
  __builtin_memcpy(&f, &b, 2);
  return float(f);
}

// ---- K7 ----------------------------------------------------------------------
// One thread per (row, block): the block's 32 values, its scale and its two
// 16-byte fragment pieces.  Rows past M (padding to 32) quantise to zeros.
__global__ __launch_bounds__(256) void k_q8_act_quant(const float *__restrict__ a, int M, int K, int m_pad,
                                                      uint4 *__restrict__ afrag, float *__restrict__ dx) {
  const int kb_n = K / 32;
  const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
  if (id >= (long long)m_pad * kb_n) return;
  const int row = int(id / kb_n), kb = int(id % kb_n);
  float v[32];
  if (row < M) {
    const float4 *p = reinterpret_cast<const float4 *>(a + size_t(row) * K + size_t(kb) * 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 f = p[i];
      v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float d = amax / 127.0f;
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) word |= (uint32_t(int(roundf(v[4 * j + e] * inv))) & 255u) << (8 * e);
    w[j] = word;
  }
  // piece (m32, kb, lane): 16 bytes of row m32*32 + lane%32, elements 16*(lane/32) ..
  const size_t base = (size_t(row >> 5) * kb_n + kb) * 64 + (row & 31);
  afrag[base] = make_uint4(w[0], w[1], w[2], w[3]);
  afrag[base + 32] = make_uint4(w[4], w[5], w[6], w[7]);
  dx[size_t(kb) * m_pad + row] = d;
}

// ---- K8 ----------------------------------------------------------------------
struct I8GemmArgs {
  const uint4 *afrag;  // [m_pad/32][kb_n][64] pieces
  const float *dx;     // [kb_n][m_pad]
  const uint8_t *w;    // Q8_0 tiled layout
  GGLayout l;
  float *c;            // [M][N]
  int M, N, m_pad, kb_n, mtiles, ntiles;
};

constexpr int TM = 64, TN = 128;

// This lane's operands for block kb: A fragment, the B fragments and scales of
// its two column tiles, and the activation scales of its 16 rows.
struct I8Stage {
  v4i a;
  v4i b[2];
  float dw[2];
  float4 dxq[4];
};

__device__ __forceinline__ void load_stage(I8Stage &s, const I8GemmArgs &g, Rsrc ar, Rsrc wr, Rsrc dr, int m32,
                                           int n0, int kb, int lane) {
  const bool in = kb < g.kb_n;
  {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(
        ar, int(in ? uint32_t(((size_t(m32) * g.kb_n + kb) * 64 + lane) * 16) : kOutside), 0, 0);
    s.a = v4i{int(v[0]), int(v[1]), int(v[2]), int(v[3])};
  }
  const int u = kb >> 3, k8 = kb & 7, hi = lane >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 32 * j + (lane & 31);
    const bool ok = in && n < g.l.tiles * 64;
    const size_t tu = size_t(n >> 6) * g.l.units + u;
    const uint32_t qoff = ok ? uint32_t(((tu * 16 + 2 * k8 + hi) * 64 + (n & 63)) * 16) : kOutside;
    const uint32_t doff = ok ? uint32_t(g.l.side1_off + (tu * 64 + (n & 63)) * 16 + 2 * k8) : kOutside;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(wr, int(qoff), 0, 0);
    s.b[j] = v4i{int(v[0]), int(v[1]), int(v[2]), int(v[3])};
    s.dw[j] = half_to_f(__builtin_amdgcn_raw_buffer_load_b16(wr, int(doff), 0, 0));
  }
  // rows 8q + 4*hi + 0..3 of the 32-row block: four consecutive scales
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t off = in ? uint32_t((size_t(kb) * g.m_pad + m32 * 32 + 8 * q + 4 * hi) * 4) : kOutside;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(dr, int(off), 0, 0);
    s.dxq[q] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
  }
}

__device__ __forceinline__ void block_step(float (&acc)[2][16], const I8Stage &s) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(s.a, s.b[j], v16i{}, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float dq[4] = {s.dxq[q].x, s.dxq[q].y, s.dxq[q].z, s.dxq[q].w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * q + r;  // lane holds C[8q + 4*(lane/32) + r][lane%32]
        acc[j][i] = fmaf(float(d[i]), dq[r] * s.dw[j], acc[j][i]);
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_q8_gemm_i8(const I8GemmArgs g) {
  const int b = blockIdx.x;
  const int xcd = b & 7, kq = b >> 3;
  const int qn = kq / g.mtiles;
  const int ntile = qn * 8 + xcd, mtile = kq - qn * g.mtiles;
  if (ntile >= g.ntiles) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m32 = mtile * (TM / 32) + (wave & 1);
  const int n0 = ntile * TN + 64 * (wave >> 1);
  const Rsrc ar = rsrc(g.afrag, size_t(g.m_pad) * g.kb_n * 32);
  const Rsrc wr = rsrc(g.w, g.l.total);
  const Rsrc dr = rsrc(g.dx, size_t(g.kb_n) * g.m_pad * 4);

  float acc[2][16];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
  // Two stages in flight: block kb + 1 loads while block kb computes.
  I8Stage s0, s1;
  load_stage(s0, g, ar, wr, dr, m32, n0, 0, lane);
  for (int kb = 0; kb < g.kb_n; kb += 2) {
    load_stage(s1, g, ar, wr, dr, m32, n0, kb + 1, lane);
    block_step(acc, s0);
    if (kb + 1 >= g.kb_n) break;
    load_stage(s0, g, ar, wr, dr, m32, n0, kb + 2, lane);
    block_step(acc, s1);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + 32 * j + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = m32 * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      if (row < g.M) g.c[size_t(row) * g.N + col] = acc[j][i];
    }
  }
}

}  // namespace

size_t q8_i8_workspace(int M, int K) {
  const int m_pad = (M + 63) / 64 * 64;
  return ((size_t(m_pad) * K + 255) & ~size_t(255)) + size_t(m_pad) * (K / 32) * 4;
}

void q8_gemm_i8_launch(const float *a, int M, int K, int N, const GGLayout &l, const void *w, void *ws, float *c,
                       hipStream_t s) {
  const int m_pad = (M + 63) / 64 * 64, kb_n = K / 32;
  auto *afrag = static_cast<uint4 *>(ws);
  auto *dx = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + ((size_t(m_pad) * K + 255) & ~size_t(255)));
  const long long threads = (long long)m_pad * kb_n;
  hipLaunchKernelGGL(k_q8_act_quant, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, a, M, K, m_pad, afrag,
                     dx);
  I8GemmArgs g;
  g.afrag = afrag;
  g.dx = dx;
  g.w = static_cast<const uint8_t *>(w);
  g.l = l;
  g.c = c;
  g.M = M;
  g.N = N;
  g.m_pad = m_pad;
  g.kb_n = kb_n;
  g.mtiles = m_pad / TM;
  g.ntiles = (N + TN - 1) / TN;
  const int grid = (g.ntiles + 7) / 8 * 8 * g.mtiles;
  hipLaunchKernelGGL(k_q8_gemm_i8, dim3(grid), dim3(256), 0, s, g);
  hip_check(hipGetLastError(), "q8 int8 gemm launch");
}

}  // namespace qnn
