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
//
// VALU economy (the bound): the MFMA results land in VGPRs (this file is
// built with the VGPR form of MFMA, so no accumulator-register reads), every
// block-dependent load offset is a scalar offset (no per-block address
// arithmetic), a block's fp16 weight scale arrives in a 4-byte word (one
// conversion, selecting the half), and the activation scales reach each lane
// through LDS.  About 51 VALU instructions per MFMA remain, against the 48
// of the epilogue itself.
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

__device__ __forceinline__ float half_to_f(uint32_t h) {
  const uint16_t b = uint16_t(h);
  _Float16 f;
  __builtin_memcpy(&f, &b, 2);
  return float(f);
}

// ---- K7 ----------------------------------------------------------------------
// Eight lanes per (row, block), four values each; a wave covers 8 consecutive
// rows of one block, so it reads 8 x 128 contiguous bytes and writes two
// 128-byte runs of fragment pieces.  The block maximum is exchanged among the
// eight lanes; each lane packs its 4 quants into one word of the row's piece.
// Rows past M (padding to 64) quantise to zeros.
__global__ __launch_bounds__(256) void k_q8_act_quant(const float *__restrict__ a, int M, int K, int m_pad,
                                                      uint32_t *__restrict__ afrag, float *__restrict__ dx) {
  const int kb_n = K / 32;
  const long long id = (long long)blockIdx.x * 256 + threadIdx.x;
  if (id >= (long long)m_pad * kb_n * 8) return;
  const int p = int(id & 7);
  const long long g = id >> 3;  // ((m32 * kb_n + kb) * 32 + r32)
  const int r32 = int(g & 31);
  const long long mk = g >> 5;
  const int kb = int(mk % kb_n), m32 = int(mk / kb_n);
  const int row = m32 * 32 + r32;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (row < M) v = *reinterpret_cast<const float4 *>(a + size_t(row) * K + size_t(kb) * 32 + 4 * p);
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
  amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
  const float d = amax / 127.0f;
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  const uint32_t word = (uint32_t(int(roundf(v.x * inv))) & 255u) | (uint32_t(int(roundf(v.y * inv))) & 255u) << 8 |
                        (uint32_t(int(roundf(v.z * inv))) & 255u) << 16 |
                        (uint32_t(int(roundf(v.w * inv))) & 255u) << 24;
  // piece (m32, kb, lane): 16 bytes of row m32*32 + lane%32, elements 16*(lane/32) ..
  const size_t piece = (size_t(m32) * kb_n + kb) * 64 + r32 + 32 * (p >> 2);
  afrag[piece * 4 + (p & 3)] = word;
  if (p == 0) dx[size_t(kb) * m_pad + row] = d;
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

constexpr int TM = 64;
constexpr int NJ = 2;      // 32-column MFMA tiles per wave (one tile per wave ran 10% slower: more A and
                           // scale traffic per MFMA outweighs the extra waves)
constexpr int kDepth = 4;  // blocks of A and B fragments in flight per wave

// This lane's matrix operands for one block: the A fragment, the B fragments
// of its NJ column tiles and the 4-byte words holding their fp16 scales (low
// half for even blocks).
struct I8Stage {
  v4i a;
  v4i b[NJ];
  uint32_t dw[NJ];
};
// Per-lane parts of the buffer offsets; the block-dependent parts are wave
// uniform and go in the scalar offset.  Every offset stays inside its buffer
// (columns past the layout are clamped, blocks past the end are clamped by
// the caller), so no load relies on the range check.
struct I8Offsets {
  uint32_t a, b[NJ], d[NJ];
};

__device__ __forceinline__ void load_ab(I8Stage &s, Rsrc ar, Rsrc wr, const I8Offsets &o, int kb) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(ar, int(o.a), kb * 1024, 0);
  s.a = v4i{int(v[0]), int(v[1]), int(v[2]), int(v[3])};
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const auto w = __builtin_amdgcn_raw_buffer_load_b128(wr, int(o.b[j]), kb * 2048, 0);
    s.b[j] = v4i{int(w[0]), int(w[1]), int(w[2]), int(w[3])};
    s.dw[j] = __builtin_amdgcn_raw_buffer_load_b32(wr, int(o.d[j]), (kb >> 3) * 1024 + (kb & 6) * 2, 0);
  }
}

// Activation scales go through LDS, per wave: the wave's 32 rows x kDepth
// blocks are one 8-byte load per lane, issued a group of blocks ahead and
// written to the wave's own LDS slot at the top of the group that uses them
// (a wave's own LDS write and reads stay in order: no barrier).  Each lane
// then reads its 16 rows per block as 4 x 16 bytes (broadcast within each
// half-wave).  Held as registers, the same scales would take 16 VGPRs per
// block in flight.
static_assert(kDepth == 4, "a group's scales are 32 rows x 4 blocks, two floats per lane");

__device__ __forceinline__ float2 load_scales(Rsrc dr, uint32_t vx, int m_pad, int kb0, int last, int lane) {
  kb0 = min(kb0, last);
  const int blk = min(lane >> 4, last - kb0);  // blocks past the end reload the last one (never used)
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(dr, int(vx + uint32_t(blk * m_pad * 4)), kb0 * m_pad * 4, 0);
  return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

__device__ __forceinline__ void block_step(float (&acc)[NJ][16], const I8Stage &s, const float4 *xs, int hi,
                                           bool odd) {
  float dw[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) dw[j] = half_to_f(odd ? s.dw[j] >> 16 : s.dw[j]);
  v16i d[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) d[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(s.a, s.b[j], v16i{}, 0, 0, 0);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 x = xs[2 * q + hi];  // rows 8q + 4*hi + 0..3 of the wave's 32
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float dq[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * q + r;  // lane holds C[8q + 4*(lane/32) + r][lane%32]
        acc[j][i] = fmaf(float(d[j][i]), dq[r] * dw[j], acc[j][i]);
      }
    }
  }
}

// A workgroup computes 64 rows x 64*NJ columns: wave w takes rows 32*(w & 1)
// and NJ column tiles of 32 from 32*NJ*(w >> 1).
__global__ __launch_bounds__(256) void k_q8_gemm_i8(const I8GemmArgs g) {
  __shared__ float4 xs_all[4][2][kDepth][8];  // [wave][slot][block][32 rows / 4]
  const int b = blockIdx.x;
  const int xcd = b & 7, kq = b >> 3;
  const int qn = kq / g.mtiles;
  const int ntile = qn * 8 + xcd, mtile = kq - qn * g.mtiles;
  if (ntile >= g.ntiles) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m32 = mtile * (TM / 32) + (wave & 1);
  const int n0 = ntile * 64 * NJ + 32 * NJ * (wave >> 1);
  const int hi = lane >> 5;
  const Rsrc ar = rsrc(g.afrag, size_t(g.m_pad) * g.kb_n * 32);
  const Rsrc wr = rsrc(g.w, g.l.total);
  const Rsrc dr = rsrc(g.dx, size_t(g.kb_n) * g.m_pad * 4);
  float2 *xw = reinterpret_cast<float2 *>(&xs_all[wave][0][0][0]);  // this wave's two slots

  I8Offsets o;
  o.a = uint32_t((size_t(m32) * g.kb_n * 64 + lane) * 16);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = min(n0 + 32 * j + (lane & 31), g.l.tiles * 64 - 1);
    const size_t t0 = size_t(n >> 6) * g.l.units;  // tile's first unit
    o.b[j] = uint32_t(((t0 * 16 + hi) * 64 + (n & 63)) * 16);
    o.d[j] = uint32_t(g.l.side1_off + (t0 * 64 + (n & 63)) * 16);
  }
  // lane l loads rows 2 * (l % 16) .. + 1 of block l / 16 of a group
  const uint32_t vx = uint32_t((m32 * 32 + 2 * (lane & 15)) * 4);

  float acc[NJ][16];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
  const int last = g.kb_n - 1;
  // In flight at the top of each group: that group's scales, then its kDepth
  // blocks of A and B (the same order as the loop leaves them; the
  // scheduling barriers keep it, so the wait counts at the loop head need not
  // be conservative).
  float2 hx = load_scales(dr, vx, g.m_pad, 0, last, lane);
  __builtin_amdgcn_sched_barrier(0);
  I8Stage s[kDepth];
#pragma unroll
  for (int p = 0; p < kDepth; ++p) {
    load_ab(s[p], ar, wr, o, min(p, last));
    __builtin_amdgcn_sched_barrier(0);
  }

  const int kb_main = g.kb_n - g.kb_n % kDepth;
  int slot = 0;
  for (int kb = 0; kb < kb_main; kb += kDepth) {
    xw[slot * 64 + lane] = hx;  // [block lane/16][rows 2*(lane%16) ..]
    hx = load_scales(dr, vx, g.m_pad, kb + kDepth, last, lane);
    __builtin_amdgcn_sched_barrier(0);
    const float4 *xc = &xs_all[wave][slot][0][0];
#pragma unroll
    for (int p = 0; p < kDepth; ++p) {
      block_step(acc, s[p], xc + p * 8, hi, p & 1);
      load_ab(s[p], ar, wr, o, min(kb + p + kDepth, last));
      __builtin_amdgcn_sched_barrier(0);
    }
    slot ^= 1;
  }
  // The last kb_n % kDepth blocks sit in s[0 ..], their scales in hx.
  if (kb_main < g.kb_n) {
    xw[slot * 64 + lane] = hx;
    const float4 *xc = &xs_all[wave][slot][0][0];
#pragma unroll
    for (int p = 0; p < kDepth - 1; ++p)
      if (kb_main + p < g.kb_n) block_step(acc, s[p], xc + p * 8, hi, p & 1);
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = n0 + 32 * j + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = m32 * 32 + 8 * (i >> 2) + 4 * hi + (i & 3);
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
  // Every buffer offset of the GEMM is a 32-bit byte offset.
  if (l.total > 0xFFFFFFFFull || size_t(m_pad) * K > 0xFFFFFFFFull)
    fail(QNN_E_NOT_SUPPORTED, "the int8-activation GEMM takes weights and activations below 4 GiB");
  const long long threads = (long long)m_pad * kb_n * 8;
  hipLaunchKernelGGL(k_q8_act_quant, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, a, M, K, m_pad,
                     reinterpret_cast<uint32_t *>(afrag), dx);
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
  g.ntiles = (N + 64 * NJ - 1) / (64 * NJ);
  const int grid = (g.ntiles + 7) / 8 * 8 * g.mtiles;
  hipLaunchKernelGGL(k_q8_gemm_i8, dim3(grid), dim3(256), 0, s, g);
  hip_check(hipGetLastError(), "q8 int8 gemm launch");
}

}  // namespace qnn
