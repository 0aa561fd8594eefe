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
// Each block needs its own pair of scales per output, so the epilogue, not the
// int8 matrix work, is the cost: at the cfg5 shape 512 x 12288 x 96 blocks
// there are 604 M (output, block) pairs against 7.7 us of int8 MFMA work.  The
// scale products dx[m] * dw[n] go to the fp32 matrix cores as outer products,
// two blocks per instruction (v_mfma_f32_32x32x1_2b_f32), which leaves the
// VALU two operations per output and block (convert, fma).
//
// Tiling: a 256-thread workgroup computes 64 rows x 192 columns; wave w takes
// rows 32 * (w & 1) and columns 96 * (w >> 1) as three 32 x 32 MFMA tiles.
// Activations come pre-arranged in MFMA fragment order (16 bytes per lane and
// block, one coalesced 1 KiB load per 32 rows); weight fragments are read
// straight from the tiled Q8_0 layout (lane l: row l % 32 of the tile, the
// 16 quants of half l / 32 of the block: 512 contiguous bytes per half).  All
// M-tiles of an N-tile share blockIdx % 8, so they run on one XCD and the
// weights come from HBM once.
//
// VALU economy: the MFMA results land in VGPRs (this file is built with the
// VGPR form of MFMA, so no accumulator-register reads), every block-dependent
// load offset is a scalar offset (no per-block address arithmetic), and a
// block pair's fp16 weight scales arrive in one 4-byte word (each half-wave
// converts its half).  About 33 VALU instructions per int8 MFMA remain,
// against the 32 of the convert-and-fma epilogue itself.
#include "qnn_internal.h"
#include "qnn_lanes.h"

namespace qnn {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

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
  amax = fmaxf(amax, dev::xor_lanes<1>(amax));  // the eight lanes of the block
  amax = fmaxf(amax, dev::xor_lanes<2>(amax));
  amax = fmaxf(amax, dev::xor_lanes<4>(amax));
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
constexpr int NJ = 3;      // 32-column MFMA tiles per wave: fewer A and scale bytes per MFMA (1 -> 2 -> 3
                           // tiles: 87 -> 65 -> 61 us at cfg5) outweigh the waves lost (5 -> 3 -> 2 per SIMD)
constexpr int kDepth = 4;  // blocks of A and B fragments in flight per wave

// This lane's matrix operands for one block: the A fragment, the B fragments
// of its NJ column tiles, the 4-byte words holding their fp16 scales (low
// half for even blocks) and the activation scale of its row (lane % 32).
struct I8Stage {
  v4i a;
  v4i b[NJ];
  uint32_t dw[NJ];
  float dx;
};
// Per-lane parts of the buffer offsets; the block-dependent parts are wave
// uniform and go in the scalar offset.  Every offset stays inside its buffer
// (columns past the layout are clamped, blocks past the end are clamped by
// the caller), so no load relies on the range check.
struct I8Offsets {
  uint32_t a, b[NJ], d[NJ], x;
};

// Even stages also load the pair's scales: the word with blocks kb, kb + 1's
// fp16 weight scales and, per lane, the activation scale of row lane % 32 in
// block kb + lane / 32.
template <bool SCALES>
__device__ __forceinline__ void load_ab(I8Stage &s, Rsrc ar, Rsrc wr, Rsrc dr, const I8Offsets &o, int kb,
                                        int m_pad) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(ar, int(o.a), kb * 1024, 0);
  s.a = v4i{int(v[0]), int(v[1]), int(v[2]), int(v[3])};
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const auto w = __builtin_amdgcn_raw_buffer_load_b128(wr, int(o.b[j]), kb * 2048, 0);
    s.b[j] = v4i{int(w[0]), int(w[1]), int(w[2]), int(w[3])};
    if (SCALES) s.dw[j] = __builtin_amdgcn_raw_buffer_load_b32(wr, int(o.d[j]), (kb >> 3) * 1024 + (kb & 6) * 2, 0);
  }
  if (SCALES) s.dx = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(dr, int(o.x), kb * m_pad * 4, 0));
}

// Two consecutive blocks (kb even, kb + 1): the scale products dx[m] * dw[n]
// of both 32 x 32 tiles are formed on the fp32 matrix cores as one
// two-block outer product (v_mfma_f32_32x32x1_2b_f32: lanes 0..31 hold block
// kb's scales, lanes 32..63 block kb + 1's, and each product is one rounded
// multiply, the value a VALU multiply gives), in the register layout of the
// int32 tiles.  The VALU is left with the conversion and the fma: two
// operations per output and block instead of three.  With `second` false
// (an odd block count's last block) only block kb is accumulated.
__device__ __forceinline__ void block_pair(float (&acc)[NJ][16], const I8Stage &s0, const I8Stage &s1, int hi,
                                           bool second) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float wb = half_to_f(s0.dw[j] >> (16 * hi));  // the word holds blocks kb (low) and kb + 1
    const v32f pr = __builtin_amdgcn_mfma_f32_32x32x1f32(s0.dx, wb, v32f{}, 0, 0, 0);
    const v16i d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(s0.a, s0.b[j], v16i{}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i)  // lane holds C[8 (i / 4) + 4 (lane / 32) + i % 4][lane % 32]
      acc[j][i] = fmaf(float(d0[i]), pr[i], acc[j][i]);
    if (second) {
      const v16i d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(s1.a, s1.b[j], v16i{}, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[j][i] = fmaf(float(d1[i]), pr[16 + i], acc[j][i]);
    }
  }
}

// A workgroup computes 64 rows x 64*NJ columns: wave w takes rows 32*(w & 1)
// and NJ column tiles of 32 from 32*NJ*(w >> 1).
__global__ __launch_bounds__(256) void k_q8_gemm_i8(const I8GemmArgs g) {
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
  // One block past the last is part of the workspace: a pair that starts at
  // the last block reads its (unused) second scales there.
  const Rsrc dr = rsrc(g.dx, size_t(g.kb_n + 1) * g.m_pad * 4);

  I8Offsets o;
  o.a = uint32_t((size_t(m32) * g.kb_n * 64 + lane) * 16);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = min(n0 + 32 * j + (lane & 31), g.l.tiles * 64 - 1);
    const size_t t0 = size_t(n >> 6) * g.l.units;  // tile's first unit
    o.b[j] = uint32_t(((t0 * 16 + hi) * 64 + (n & 63)) * 16);
    o.d[j] = uint32_t(g.l.side1_off + (t0 * 64 + (n & 63)) * 16);
  }
  o.x = uint32_t((m32 * 32 + (lane & 31) + hi * g.m_pad) * 4);

  float acc[NJ][16];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
  const int last = g.kb_n - 1;
  // kDepth blocks of operands in flight at the top of each group (the
  // scheduling barriers keep the issue order, so the wait counts at the loop
  // head need not be conservative).
  I8Stage s[kDepth];
#pragma unroll
  for (int p = 0; p < kDepth; p += 2) {
    load_ab<true>(s[p], ar, wr, dr, o, min(p, last), g.m_pad);
    load_ab<false>(s[p + 1], ar, wr, dr, o, min(p + 1, last), g.m_pad);
    __builtin_amdgcn_sched_barrier(0);
  }

  const int kb_main = g.kb_n - g.kb_n % kDepth;
  for (int kb = 0; kb < kb_main; kb += kDepth) {
#pragma unroll
    for (int p = 0; p < kDepth; p += 2) {
      block_pair(acc, s[p], s[p + 1], hi, true);
      load_ab<true>(s[p], ar, wr, dr, o, min(kb + p + kDepth, last), g.m_pad);
      load_ab<false>(s[p + 1], ar, wr, dr, o, min(kb + p + 1 + kDepth, last), g.m_pad);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // The last kb_n % kDepth blocks sit in s[0 ..].
#pragma unroll
  for (int p = 0; p < kDepth; p += 2)
    if (kb_main + p < g.kb_n) block_pair(acc, s[p], s[p + 1], hi, kb_main + p + 1 < g.kb_n);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = n0 + 32 * j + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = m32 * 32 + 8 * (i >> 2) + 4 * hi + (i & 3);
      if (row < g.M) __builtin_nontemporal_store(acc[j][i], &g.c[size_t(row) * g.N + col]);  // streaming: see qnn_gemm.hip
    }
  }
}

}  // namespace

size_t q8_i8_workspace(int M, int K) {
  const int m_pad = (M + 63) / 64 * 64;
  return ((size_t(m_pad) * K + 255) & ~size_t(255)) + size_t(m_pad) * (K / 32 + 1) * 4;
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
