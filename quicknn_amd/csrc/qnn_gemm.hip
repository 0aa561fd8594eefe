// qnn_gemm.hip -- multi-row GGUF Q8_0 projection (prefill GEMM) on fp16 MFMA.
//
// Replaces TQNNGPUContext.Linear with Rows > 1 on a Q8_0 weight
// (Context.Implementation.inc:852-883 -> gemm.comp:27-44, :75-105: an fp32
// SIMT GEMM that decodes every weight element into its LDS tile).
//     C[m][n] = sum_k A[m][k] * W[n][k],   W[n][k] = d_b * q_k  (GGUFValue, exact in fp32)
//
// Operands run through v_mfma_f32_32x32x16_f16 in fp16, accumulated in fp32:
//   * A is scaled per row by an exact power of two 2^-ea[m] (max |A[m][.]| in
//     (2^13, 2^14]) and rounded once to fp16;
//   * W is rounded once to fp16 as fp16(q * d * 2^-ew[n]), with the per-row
//     power of two ew[n] taken at upload (max |d*q| of the row in (2^13, 2^14]);
//   * C = acc * 2^(ea[m] + ew[n]).
// fp16 keeps 11 significant bits: the normwise error at the cfg5 shape is
// ~3e-4 (an int8 activation pass would give ~5e-3, bf16 ~2e-3).
//
// Tiling.  A workgroup computes (32 * MB * NW) x 96 of C with NW waves of
// (32 * MB) x 96 (MB x 3 MFMA tiles of 32 x 32): 256 x 96 as 8 waves of one
// block at prefill shapes, 128 x 96 as 4 waves below.  A is prepared once per call in MFMA
// fragment order (1 KiB per 32 rows x 16 k, one 16-byte piece per lane), so a
// wave loads its A fragments straight from L2 with fully coalesced 16-byte
// loads.  The 96 weight rows of a K-step are decoded once per workgroup into a
// double-buffered LDS tile (fp16, rows padded by 16 bytes: conflict-free
// ds_read_b128) that all four waves read.  All M-tiles of an N-tile run on
// one XCD, so the weight bytes are fetched from HBM once.  Loads run three
// K-tiles deep (registers), since one K-tile of MFMA work is shorter than a
// load's latency under load.
#include <type_traits>

#include "qnn_internal.h"
#include "qnn_lanes.h"

namespace qnn {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BN = 96, BK = 64, LDB = BK + 8;  // LDB: halfs per LDS weight row
// Workgroup tile: NW waves x MB 32-row blocks of C (BM = 32 * MB * NW rows) by BN columns.

__device__ __forceinline__ float half_bits_to_f(uint32_t h) {
  const uint16_t b = uint16_t(h);
  _Float16 f;
  __builtin_memcpy(&f, &b, 2);
  return float(f);
}

// ---- activation preparation ------------------------------------------------
// One launch: workgroup b owns rows 4b .. 4b + 3 of A (m_pad rows in all),
// four waves per row.  A row's 256 threads take its groups of 8 columns
// g = t, t + 256, ...: each thread requests its first AP_HOLD groups at once
// and keeps them in registers (the whole row up to K = 8192), takes ea[m]
// from max |A[m][.]| (range_exp; the four waves meet in LDS), then writes
// the fp16 values A·2^-ea (exact scaling, one RNE rounding) as the fragments
// of v_mfma_f32_32x32x16_f16's A operand: piece (m32, ks, lane) = 8 halfs
// A[m32*32 + lane%32][ks*16 + 8*(lane/32) + 0..7], so the row's group g goes
// to piece (m / 32, g / 2) at lane m % 32 + 32 (g % 2).  Groups past the held
// ones are read twice (once for the maximum, once for the values).  The four
// rows of a workgroup fill the same 64-byte segments together (one row per
// workgroup wrote every segment in four visits: twice the bytes).  Rows past
// M and columns past K give exponent 0 and zero pieces.
constexpr int AP_HOLD = 4;
__global__ __launch_bounds__(1024) void k_act_prep(const float *__restrict__ a, int M, int K, int ksteps,
                                                   int *__restrict__ ea, uint4 *__restrict__ frag) {
  __shared__ float red[4][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, rw = wave >> 2, part = wave & 3;
  const int t = part * 64 + lane;  // thread of the row, 0 .. 255
  const int row = blockIdx.x * 4 + rw;
  const bool in = row < M;
  const float *r = a + size_t(in ? row : 0) * K;
  const bool vec = (K & 3) == 0;
  const int groups = 2 * ksteps;  // groups of 8 columns, K padded to 16
  auto load8 = [&](int g, float (&v)[8]) {
    const int k0 = 8 * g;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    if (!in) return;
    if (vec && k0 + 8 <= K) {
      const float4 x0 = *reinterpret_cast<const float4 *>(r + k0), x1 = *reinterpret_cast<const float4 *>(r + k0 + 4);
      v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k0 + i < K) v[i] = r[k0 + i];
    }
  };
  auto vmax = [](float m, const float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    return m;
  };
  float held[AP_HOLD][8];
#pragma unroll
  for (int c = 0; c < AP_HOLD; ++c) {
    if (t + 256 * c < groups) {
      load8(t + 256 * c, held[c]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) held[c][i] = 0.0f;
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < AP_HOLD; ++c) amax = vmax(amax, held[c]);
  for (int g = t + 256 * AP_HOLD; g < groups; g += 256) {
    float v[8];
    load8(g, v);
    amax = vmax(amax, v);
  }
  amax = dev::wave_max_xor(amax);
  if (lane == 0) red[rw][part] = amax;
  __syncthreads();
  const int e = range_exp(fmaxf(fmaxf(red[rw][0], red[rw][1]), fmaxf(red[rw][2], red[rw][3])));
  if (t == 0) ea[row] = e;
  const float sc = ldexpf(1.0f, -e);
  uint4 *dst = frag + size_t(row >> 5) * ksteps * 64 + (row & 31);
  auto put = [&](int g, float (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] *= sc;  // exact: power of two
    dst[size_t(g >> 1) * 64 + 32 * (g & 1)] =
        make_uint4(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), pack_h2(v[4], v[5]), pack_h2(v[6], v[7]));
  };
#pragma unroll
  for (int c = 0; c < AP_HOLD; ++c)
    if (t + 256 * c < groups) put(t + 256 * c, held[c]);
  for (int g = t + 256 * AP_HOLD; g < groups; g += 256) {
    float v[8];
    load8(g, v);
    put(g, v);
  }
}

// ---- weight row exponents (at upload) --------------------------------------
__global__ void k_q8_rowexp(GGLayout l, uint8_t *__restrict__ w) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= l.tiles * 64) return;
  const int t = row >> 6, r = row & 63;
  const uint8_t *side = w + l.side1_off;
  float dmax = 0.0f;
  for (int u = 0; u < l.units; ++u) {
    const uint4 ds = *reinterpret_cast<const uint4 *>(side + ((size_t(t) * l.units + u) * 64 + r) * 16);
    const uint32_t dw[4] = {ds.x, ds.y, ds.z, ds.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dmax = fmaxf(dmax, fabsf(half_bits_to_f(dw[j] & 0xFFFFu)));
      dmax = fmaxf(dmax, fabsf(half_bits_to_f(dw[j] >> 16)));
    }
  }
  reinterpret_cast<int *>(w + l.rowexp_off)[row] = range_exp(dmax * 127.0f);
}

// ---- GEMM ---------------------------------------------------------------------
struct GemmArgs {
  const uint4 *afrag;  // [m_pad/32][ksteps][64] pieces
  const int *ea;       // [m_pad]
  const uint8_t *w;    // Q8_0 tiled layout
  GGLayout l;
  float *c;            // [M][N]
  int M, N, ksteps, ktiles, mtiles, ntiles;
};

// Weight loader: threads 0..191 each own (row i = t/2, block h = t%2) of the
// 96 x 64 K-step: two 16-byte quant pieces and the block's fp16 scale.
struct BRaw {
  uint4 q0, q1;
  uint32_t d;
};

// Buffer loads without branches, so the compiler can count them across the
// software pipeline: threads past the 96 rows and blocks past the matrix read
// at an offset beyond the buffer, which returns zeros.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(uint32_t(min(bytes, size_t(0xFFFFFFFFu)))),
                                           0x00020000);
}
__device__ __forceinline__ uint4 ld128(Rsrc r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
constexpr uint32_t kOutside = 0xFFFFFFF0u;

__device__ __forceinline__ void load_b(BRaw &b, const GemmArgs &g, Rsrc wr, int ntile, int kt, int tid) {
  const int n = ntile * BN + (tid >> 1);
  const int kb = kt * 2 + (tid & 1);  // 32-element block
  const bool in = tid < 2 * BN && n < g.l.tiles * 64 && kb < g.l.units * 8;
  const int t = n >> 6, r = n & 63, u = kb >> 3, k8 = kb & 7;
  const size_t tu = size_t(t) * g.l.units + u;
  const uint32_t qoff = in ? uint32_t(((tu * 16 + 2 * k8) * 64 + r) * 16) : kOutside;
  const uint32_t doff = in ? uint32_t(g.l.side1_off + (tu * 64 + r) * 16 + 2 * k8) : kOutside;
  b.q0 = ld128(wr, qoff);
  b.q1 = ld128(wr, qoff + (qoff == kOutside ? 0u : 1024u));
  b.d = __builtin_amdgcn_raw_buffer_load_b16(wr, int(doff), 0, 0);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_b(_Float16 (*bs)[LDB], const BRaw &b, float scale, int tid) {
  if (tid >= 2 * BN) return;
  const float ds = half_bits_to_f(b.d) * scale;  // d * 2^-ew (exact)
  const uint32_t qw[8] = {b.q0.x, b.q0.y, b.q0.z, b.q0.w, b.q1.x, b.q1.y, b.q1.z, b.q1.w};
  uint32_t hw[16];
  if (fabsf(ds) >= 6.103515625e-05f) {
    // ds is an fp16 normal, so fp16 arithmetic gives the same single rounding
    // RNE(q * ds) as the fp32 product below: each byte q goes under the fp16
    // exponent of 1024 as (q + 128) (v_perm), x - 1152 = q exactly, and one
    // packed fp16 multiply rounds q * ds.
    const _Float16 dh = _Float16(ds);  // exact
    const half2v dsh = {dh, dh}, off = {_Float16(1152.0f), _Float16(1152.0f)};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t u = qw[i] ^ 0x80808080u;
      const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // q0 + 1152, q1 + 1152
      const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // q2 + 1152, q3 + 1152
      half2v a, c;
      __builtin_memcpy(&a, &lo, 4);
      __builtin_memcpy(&c, &hi, 4);
      a = (a - off) * dsh;
      c = (c - off) * dsh;
      __builtin_memcpy(&hw[2 * i], &a, 4);
      __builtin_memcpy(&hw[2 * i + 1], &c, 4);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q0 = int(int8_t(qw[i] & 255u)), q1 = int(int8_t((qw[i] >> 8) & 255u));
      const int q2 = int(int8_t((qw[i] >> 16) & 255u)), q3 = int(int8_t(qw[i] >> 24));
      hw[2 * i] = pack_h2(float(q0) * ds, float(q1) * ds);
      hw[2 * i + 1] = pack_h2(float(q2) * ds, float(q3) * ds);
    }
  }
  uint4 *dst = reinterpret_cast<uint4 *>(&bs[tid >> 1][(tid & 1) * 32]);
#pragma unroll
  for (int j = 0; j < 4; ++j) dst[j] = make_uint4(hw[4 * j], hw[4 * j + 1], hw[4 * j + 2], hw[4 * j + 3]);
}

template <int MB, int NW>
__global__ __launch_bounds__(NW * 64) void k_q8_gemm(const GemmArgs g) {
  constexpr int BM = 32 * MB * NW;
  const int b = blockIdx.x;
  // XCD-aware: the M-tiles of one N-tile have the same blockIdx % 8, so with the
  // device's usual round-robin dealing they share an XCD and its L2.
  const int xcd = b & 7, kq = b >> 3;
  const int q = kq / g.mtiles;
  const int ntile = q * 8 + xcd, mtile = kq - q * g.mtiles;
  if (ntile >= g.ntiles) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  __shared__ __attribute__((aligned(16))) _Float16 bs[2][BN][LDB];
  __shared__ float wscale[BN];
  if (tid < BN) {
    const int n = ntile * BN + tid;
    const int e = n < g.l.tiles * 64 ? reinterpret_cast<const int *>(g.w + g.l.rowexp_off)[n] : 0;
    wscale[tid] = ldexpf(1.0f, -e);
  }
  const int m32 = (mtile * BM + wave * 32 * MB) >> 5;  // first 32-row block of this wave
  // A fragments: piece (m32 + mb, ks) of this lane at byte ((m32 + mb) * ksteps + ks) * 1024 + lane * 16;
  // pieces past the last K-step read zeros.
  const Rsrc ar = rsrc(g.afrag, size_t(g.mtiles) * MB * NW * g.ksteps * 1024);
  const Rsrc wr = rsrc(g.w, g.l.total);
  uint32_t aoff[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) aoff[mb] = uint32_t((size_t(m32 + mb) * g.ksteps) * 1024 + lane * 16);

  f32x16 acc[MB][3];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Software pipeline: the raw weights and the A fragments of K-tile kt + 2
  // are requested while K-tile kt runs on the MFMAs and kt + 1 is decoded into
  // the other LDS buffer, so each load has two K-tiles of work (~0.6 us) to
  // arrive in.  Stages live in registers, indexed statically (kt % 3).
  constexpr int D = 3;
  BRaw braw[D];
  uint4 a[D][MB][4];
  auto load_stage = [&](auto S_, int kt) {
    constexpr int S = decltype(S_)::value;
    load_b(braw[S], g, wr, ntile, kt, tid);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int kk = kt * 4 + ks;
        a[S][mb][ks] = ld128(ar, kk < g.ksteps ? aoff[mb] + uint32_t(kk) * 1024u : kOutside);
      }
  };
  load_stage(std::integral_constant<int, 0>(), 0);
  load_stage(std::integral_constant<int, 1>(), 1);
  __syncthreads();  // wscale
  store_b(bs[0], braw[0], tid < 2 * BN ? wscale[tid >> 1] : 0.0f, tid);
  __syncthreads();

  auto iter = [&](auto S_, int kt) {
    constexpr int S = decltype(S_)::value;
    constexpr int S1 = (S + 1) % D, S2 = (S + 2) % D;
    const int buf = kt & 1;
    load_stage(std::integral_constant<int, S2>(), kt + 2);  // past the end: zeros, unused
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      half8 bf[3];
#pragma unroll
      for (int nb = 0; nb < 3; ++nb) {
        const uint4 v = *reinterpret_cast<const uint4 *>(&bs[buf][nb * 32 + (lane & 31)][ks * 16 + 8 * (lane >> 5)]);
        __builtin_memcpy(&bf[nb], &v, 16);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        half8 af;
        __builtin_memcpy(&af, &a[S][mb][ks], 16);
#pragma unroll
        for (int nb = 0; nb < 3; ++nb) acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[nb], acc[mb][nb], 0, 0, 0);
      }
    }
    if (kt + 1 < g.ktiles) store_b(bs[buf ^ 1], braw[S1], tid < 2 * BN ? wscale[tid >> 1] : 0.0f, tid);
    __syncthreads();
  };
  for (int kt = 0; kt < g.ktiles; kt += D) {
    iter(std::integral_constant<int, 0>(), kt);
    if (kt + 1 < g.ktiles) iter(std::integral_constant<int, 1>(), kt + 1);
    if (kt + 2 < g.ktiles) iter(std::integral_constant<int, 2>(), kt + 2);
  }

  // Epilogue: lane holds C[8*(i/4) + 4*(lane/32) + i%4][lane%32] of each 32x32 tile.
  // The row and column exponents are loaded before any store of C: as far as
  // the compiler knows C may alias them, so a load after a store waits for it.
  // C is written with streaming stores: every workgroup writes its tile at the
  // same moment, and keeping the lines out of the L2 shortens that burst.
  int ear[MB][16], ewr[3];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = mtile * BM + wave * 32 * MB + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      ear[mb][i] = row < g.M ? g.ea[row] : 0;
    }
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int col = ntile * BN + nb * 32 + (lane & 31);
    ewr[nb] = col < g.N ? reinterpret_cast<const int *>(g.w + g.l.rowexp_off)[col] : 0;
  }
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int col = ntile * BN + nb * 32 + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = mtile * BM + wave * 32 * MB + mb * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row < g.M)
          __builtin_nontemporal_store(ldexpf(acc[mb][nb][i], ear[mb][i] + ewr[nb]), &g.c[size_t(row) * g.N + col]);
      }
    }
  }
}

// ---- the same product over a pre-expanded fp16 copy of the weight ----------
// The copy holds, for every weight, the fp16 value store_b decodes into LDS
// (RNE(q * d * 2^-ew[n])), laid out as v_mfma_f32_32x32x16_f16 B fragments:
// piece (n32, ks, lane) = 8 halfs W[32 n32 + lane % 32][16 ks + 8 (lane / 32) + 0..7]
// at ((n32 * ksteps + ks) * 64 + lane) * 16 bytes; rows past N and columns
// past K hold zeros.  It is made once per weight (k_q8_expand_h16) and kept
// in the weight cache beside the Q8_0 copy.
__global__ __launch_bounds__(256) void k_q8_expand_h16(GGLayout l, const uint8_t *__restrict__ w, int ksteps,
                                                       size_t pieces, uint4 *__restrict__ out) {
  const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= pieces) return;
  const int lane = int(idx & 63);
  const size_t nk = idx >> 6;
  const int ks = int(nk % ksteps), n32 = int(nk / ksteps);
  const int n = n32 * 32 + (lane & 31), k0 = ks * 16 + 8 * (lane >> 5);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (n < l.rows && k0 < l.cols) {
    const int kb = k0 >> 5, e0 = k0 & 31;
    const int t = n >> 6, r = n & 63, u = kb >> 3, k8 = kb & 7;
    const size_t tu = size_t(t) * l.units + u;
    const uint32_t dword = *reinterpret_cast<const uint32_t *>(w + l.side1_off + (tu * 64 + r) * 16 + 4 * (k8 >> 1));
    const float scale = ldexpf(1.0f, -reinterpret_cast<const int *>(w + l.rowexp_off)[n]);
    const float ds = half_bits_to_f((k8 & 1) ? (dword >> 16) : (dword & 0xFFFFu)) * scale;  // exact
    const uint2 q = *reinterpret_cast<const uint2 *>(w + ((tu * 16 + 2 * k8 + (e0 >> 4)) * 64 + r) * 16 + (e0 & 15));
    const uint32_t qw[2] = {q.x, q.y};
    uint32_t hw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = qw[i >> 1] >> (16 * (i & 1));
      hw[i] = pack_h2(float(int(int8_t(word & 255u))) * ds, float(int(int8_t((word >> 8) & 255u))) * ds);
    }
    v = make_uint4(hw[0], hw[1], hw[2], hw[3]);
  }
  out[idx] = v;
}

// Workgroup tile 128 x 192 (a 512 x 12288 product is 4 x 64 = 256
// workgroups, one per CU), four waves of 64 x 96 (2 x 3 MFMA tiles), K-tiles
// of 64.  A K-tile's fragments (A: 4 x 4 pieces, B: 6 x 4 pieces of 1 KiB)
// go from global memory straight into LDS (buffer_load ... lds: each lane's
// 16 bytes land at M0 + 16 lane, so a piece keeps its [lane] order) through
// HST stages of 40 KiB (all 160 KiB of the CU's LDS: the loads run up to
// three K-tiles ahead).  Per K-tile, one barrier: after it the K-tile's stage
// is free (every wave holds its fragments in registers) and takes the loads
// of K-tile kt + HST; then each wave reads the next K-tile's fragments (20
// pieces, 80 VGPRs) while its MFMAs run on the current ones.  Per 32 x 32
// tile the MFMAs run over K in order, as in k_q8_gemm, so C is the same, bit
// for bit.
constexpr int HBM = 128, HBN = 192, HKT = 4;  // rows, columns, K-steps (of 16) per K-tile
constexpr int HAP = HBM / 32 * HKT, HBP = HBN / 32 * HKT;  // 1 KiB pieces per K-tile: 16 + 24
constexpr int HPW = (HAP + HBP) / 4;                        // pieces each wave loads per K-tile: 10
constexpr int HST = 4;                                      // LDS stages
constexpr size_t kH16Lds = size_t(HST) * (HAP + HBP) * 1024;
static_assert(HAP % 4 == 0 && kH16Lds <= 160 * 1024, "h16 tiling");
struct H16Args {
  const uint4 *afrag;  // [m_pad / 32][ksteps][64]
  const int *ea;
  const uint4 *wfrag;  // [n_pad / 32][ksteps][64]
  const int *ew;       // [rows] weight row exponents
  float *c;            // ksplit 1: C [M][N]; else the slices' partial products [ksplit][M][N]
  int M, N, ksteps, ktiles, mtiles, ntiles, ksplit;
};

// One 1 KiB piece from global memory into LDS at `lds` (wave-uniform).  The
// compiler does not see these writes to LDS: h16_vmwait orders them.  (Its
// own LDS-DMA builtin would make it wait for every outstanding load before
// any LDS read, draining the prefetch each K-tile.)  M0 is set here before
// each load; nothing else in this kernel uses M0 (gfx950's LDS instructions
// do not read it), which the kernel's assembly shows.
__device__ __forceinline__ void h16_dma(Rsrc r, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(r),
               "s"(soff)
               : "memory");
}
// Wait until at most N of this wave's vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void h16_vmwait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

extern __shared__ uint4 h16_lds[];  // HST stages of [HAP + HBP] pieces: A [m32][ks], then B [n32][ks]

struct H16Frags {
  half8 a[HKT][2], b[HKT][3];
};

// KS: the launch slices K (g.ksplit > 1); the instance without slices keeps
// the plain N-tile mapping and loop bounds.
template <bool KS>
__global__ __launch_bounds__(256) void k_h16_gemm(const H16Args g) {
  const int b = blockIdx.x;
  // Units (N-tile, K-slice) are dealt to the XCDs in turn; the M-tiles of a
  // unit share blockIdx % 8 (an XCD, its L2, which then fetches the unit's
  // weight columns once).
  const int xcd = b & 7, kq = b >> 3;
  const int q = kq / g.mtiles, mtile = kq - q * g.mtiles, unit = q * 8 + xcd;
  if (unit >= (KS ? g.ntiles * g.ksplit : g.ntiles)) return;
  const int ntile = KS ? unit % g.ntiles : unit, ks = KS ? unit / g.ntiles : 0;
  // K-slice ks: K-tiles [kt0, kt0 + nkt).
  const int kt0 = KS ? ks * g.ktiles / g.ksplit : 0;
  const int nkt = KS ? (ks + 1) * g.ktiles / g.ksplit - kt0 : g.ktiles;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  const Rsrc ar = rsrc(g.afrag, size_t(g.mtiles) * (HBM / 32) * g.ksteps * 1024);
  const Rsrc br = rsrc(g.wfrag, size_t(g.ntiles) * (HBN / 32) * g.ksteps * 1024);
  const uint32_t lds0 = uint32_t(reinterpret_cast<uintptr_t>(h16_lds));
  // This wave loads pieces p = wave + 4 i of every K-tile: i < HAP / 4 are A pieces.
  uint32_t voff[HPW];
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    const int p = wave + 4 * i;
    if (i < HAP / 4) {
      voff[i] = uint32_t(((size_t(mtile) * (HBM / 32) + p / HKT) * g.ksteps + p % HKT) * 1024 + lane * 16);
    } else {
      const int pb = p - HAP;
      voff[i] = uint32_t(((size_t(ntile) * (HBN / 32) + pb / HKT) * g.ksteps + pb % HKT) * 1024 + lane * 16);
    }
  }
  auto dma = [&](int kt, int i) {
    const uint32_t st = lds0 + uint32_t(kt % HST) * ((HAP + HBP) * 1024u);
    h16_dma(i < HAP / 4 ? ar : br, __builtin_amdgcn_readfirstlane(st + uint32_t(wave + 4 * i) * 1024u), voff[i],
            uint32_t(kt0 + kt) * (HKT * 1024u));
  };
  // Piece r of this wave's 5 HKT per K-tile: K-step r / 5, then A rows wm*2 + 0..1, B columns wn*3 + 0..2.
  auto read1 = [&](H16Frags &f, const uint4 *st, int r) {
    const int ks = r / 5, j = r % 5;
    if (j < 2)
      __builtin_memcpy(&f.a[ks][j], &st[((wm * 2 + j) * HKT + ks) * 64 + lane], 16);
    else
      __builtin_memcpy(&f.b[ks][j - 2], &st[(HAP + (wn * 3 + j - 2) * HKT + ks) * 64 + lane], 16);
  };

  f32x16 acc[2][3];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // K-tile kt: wait for K-tile kt + 1 (this wave's pieces, then everybody's:
  // K-tile kt's stage is then free), then the 24 MFMAs of K-tile kt, each
  // followed by one read of K-tile kt + 1's fragments and every second one by
  // one load of K-tile kt + HST into kt's stage, in this order (an MFMA does
  // not wait behind the wave's memory instructions).
  auto tile = [&](auto REFILL, const H16Frags &cur, H16Frags &nxt, int kt) {
    if (decltype(REFILL)::value)
      h16_vmwait<HPW * (HST - 2)>();
    else
      h16_vmwait<0>();
    __syncthreads();
    const uint4 *st = h16_lds + ((kt + 1) % HST) * ((HAP + HBP) * 64);  // past the end: unused
#pragma unroll
    for (int j = 0; j < 6 * HKT; ++j) {
      const int ks = j / 6, mb = (j % 6) / 3, nb = j % 3;
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.a[ks][mb], cur.b[ks][nb], acc[mb][nb], 0, 0, 0);
      if (j < 5 * HKT) read1(nxt, st, j);
      if (decltype(REFILL)::value && (j & 1) && j / 2 < HPW) dma(kt + HST, j / 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int d = 0; d < HST; ++d)
    if (d < nkt)
#pragma unroll
      for (int i = 0; i < HPW; ++i) dma(d, i);
  H16Frags f0, f1;
  if (HST - 1 < nkt)
    h16_vmwait<HPW * (HST - 1)>();
  else
    h16_vmwait<0>();
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 5 * HKT; ++r) read1(f0, h16_lds, r);
  using Y = std::true_type;
  using N = std::false_type;
  int kt = 0;
  for (; kt + 1 + HST < nkt; kt += 2) {  // both K-tiles refill
    tile(Y(), f0, f1, kt);
    tile(Y(), f1, f0, kt + 1);
  }
  for (; kt < nkt; kt += 2) {
    if (kt + HST < nkt)
      tile(Y(), f0, f1, kt);
    else
      tile(N(), f0, f1, kt);
    if (kt + 1 < nkt) tile(N(), f1, f0, kt + 1);
  }

  // Epilogue: lane holds C[8*(i/4) + 4*(lane/32) + i%4][lane%32] of each 32 x 32 tile.
  // The row and column exponents are loaded before any store of C: as far as
  // the compiler knows C may alias them, so a load after a store waits for it.
  // C is written with streaming stores: every workgroup writes its tile at the
  // same moment, and keeping the lines out of the L2 shortens that burst.
  int ear[2][16], ewr[3];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = mtile * HBM + (wm * 2 + mb) * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      ear[mb][i] = row < g.M ? g.ea[row] : 0;
    }
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int col = ntile * HBN + (wn * 3 + nb) * 32 + (lane & 31);
    ewr[nb] = col < g.N ? g.ew[col] : 0;
  }
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int col = ntile * HBN + (wn * 3 + nb) * 32 + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = mtile * HBM + (wm * 2 + mb) * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row < g.M)
          __builtin_nontemporal_store(ldexpf(acc[mb][nb][i], ear[mb][i] + ewr[nb]),
                                      &g.c[(size_t(ks) * g.M + row) * g.N + col]);
      }
    }
  }
}

}  // namespace

size_t q8_h16_bytes(int rows, int cols) {
  const size_t n_pad = size_t((rows + HBN - 1) / HBN) * HBN, k_pad = size_t((cols + 63) / 64) * 64;
  return n_pad * k_pad * 2;
}

void q8_expand_h16_launch(const GGLayout &l, const void *w, void *out, hipStream_t s) {
  const int ksteps = (l.cols + 63) / 64 * 4;
  const size_t pieces = q8_h16_bytes(l.rows, l.cols) / 16;
  hipLaunchKernelGGL(k_q8_expand_h16, dim3((pieces + 255) / 256), dim3(256), 0, s, l, static_cast<const uint8_t *>(w),
                     ksteps, pieces, static_cast<uint4 *>(out));
  hip_check(hipGetLastError(), "q8 fp16 expansion");
}

Q8GemmPlan q8_h16_plan(int M, int K, int N) {
  Q8GemmPlan p;
  p.m_pad = (M + HBM - 1) / HBM * HBM;
  p.k_pad = (K + 63) / 64 * 64;
  p.ksteps = p.k_pad / 16;
  p.mtiles = p.m_pad / HBM;
  p.ntiles = (N + HBN - 1) / HBN;
  p.frag_bytes = size_t(p.m_pad) * p.k_pad * 2;
  p.exp_bytes = size_t(p.m_pad) * 4;
  return p;
}

// C = the K-slices' partial products summed in slice order (float4 pieces).
__global__ __launch_bounds__(256) void k_sum_kslices(float4 *__restrict__ c, const float4 *__restrict__ part,
                                                     size_t count4, int slices) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count4) return;
  float4 v = part[i];
  for (int s = 1; s < slices; ++s) {
    const float4 o = part[size_t(s) * count4 + i];
    v.x += o.x;
    v.y += o.y;
    v.z += o.z;
    v.w += o.w;
  }
  c[i] = v;
}

// K-slices for a grid of few tiles: as many as keep every workgroup of the
// launch resident at once.  The kernel takes a CU's whole LDS (one workgroup
// per CU), and an XCD (32 CUs) holds ceil(ntiles * ksplit / 8) units of
// mtiles workgroups; at least 8 K-tiles per slice, at most 8 slices.
int h16_ksplit(const Q8GemmPlan &p, int N) {
  const int ktiles = p.ksteps / HKT;
  if (N % 4 != 0) return 1;
  int best = 1;
  for (int s = 2; s <= 8 && ktiles / s >= 8; ++s)
    if ((p.ntiles * s + 7) / 8 * p.mtiles <= 32) best = s;
  return best;
}

void q8_h16_gemm_launch(const Q8GemmPlan &p, const float *a, int M, int K, int N, const int *ew, const void *w16,
                        void *frag, int *ea, float *c, hipStream_t s, int ksplit, float *part) {
  hipLaunchKernelGGL(k_act_prep, dim3(p.m_pad / 4), dim3(1024), 0, s, a, M, K, p.ksteps, ea, static_cast<uint4 *>(frag));
  H16Args g;
  g.afrag = static_cast<const uint4 *>(frag);
  g.ea = ea;
  g.wfrag = static_cast<const uint4 *>(w16);
  g.ew = ew;
  g.c = ksplit > 1 ? part : c;
  g.M = M;
  g.N = N;
  g.ksteps = p.ksteps;
  g.ktiles = p.ksteps / HKT;
  g.mtiles = p.mtiles;
  g.ntiles = p.ntiles;
  g.ksplit = std::max(1, ksplit);
  const int grid = (p.ntiles * g.ksplit + 7) / 8 * 8 * p.mtiles;
  static const hipError_t attr = [] {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_h16_gemm<false>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, int(kH16Lds));
    return e != hipSuccess ? e
                           : hipFuncSetAttribute(reinterpret_cast<const void *>(&k_h16_gemm<true>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, int(kH16Lds));
  }();
  hip_check(attr, "fp16-copy gemm LDS size");
  if (g.ksplit > 1)
    hipLaunchKernelGGL(k_h16_gemm<true>, dim3(grid), dim3(256), kH16Lds, s, g);
  else
    hipLaunchKernelGGL(k_h16_gemm<false>, dim3(grid), dim3(256), kH16Lds, s, g);
  hip_check(hipGetLastError(), "q8 fp16-copy gemm launch");
  if (g.ksplit > 1) {
    const size_t count4 = size_t(M) * N / 4;
    hipLaunchKernelGGL(k_sum_kslices, dim3((count4 + 255) / 256), dim3(256), 0, s, reinterpret_cast<float4 *>(c),
                       reinterpret_cast<const float4 *>(part), count4, g.ksplit);
    hip_check(hipGetLastError(), "gemm K-slice sum launch");
  }
}

void q8_rowexp_launch(const GGLayout &l, void *w, hipStream_t s) {
  const int rows = l.tiles * 64;
  hipLaunchKernelGGL(k_q8_rowexp, dim3((rows + 255) / 256), dim3(256), 0, s, l, static_cast<uint8_t *>(w));
  hip_check(hipGetLastError(), "q8 row exponents");
}

Q8GemmPlan q8_gemm_plan(int M, int K, int N) {
  Q8GemmPlan p;
  // Prefill shapes (M >= 256): workgroup tile 256 x 96 as 8 waves of one
  // 32-row block, so two waves per SIMD hide each other's waits (cfg5: 71.6 us
  // against 76.8 for 4 waves of two blocks, the same tile; the weight decode
  // per tile is shared by all of them).  Fewer rows: 128 x 96 as 4 waves.
  // QNN_GEMM_NW / QNN_GEMM_MB override.
  p.nw = tuning().gemm_nw;
  if (p.nw != 4 && p.nw != 8) p.nw = M >= 256 ? 8 : 4;
  p.mb = tuning().gemm_mb;
  if (p.mb != 1 && p.mb != 2) p.mb = 1;
  const int BM = 32 * p.mb * p.nw;
  p.m_pad = (M + BM - 1) / BM * BM;
  p.k_pad = (K + BK - 1) / BK * BK;
  p.ksteps = p.k_pad / 16;
  p.mtiles = p.m_pad / BM;
  p.ntiles = (N + BN - 1) / BN;
  p.frag_bytes = size_t(p.m_pad) * p.k_pad * 2;
  p.exp_bytes = size_t(p.m_pad) * 4;
  return p;
}

void q8_gemm_launch(const Q8GemmPlan &p, const float *a, int M, int K, int N, const GGLayout &l, const void *w,
                    void *frag, int *ea, float *c, hipStream_t s) {
  hipLaunchKernelGGL(k_act_prep, dim3(p.m_pad / 4), dim3(1024), 0, s, a, M, K, p.ksteps, ea, static_cast<uint4 *>(frag));
  GemmArgs g;
  g.afrag = static_cast<const uint4 *>(frag);
  g.ea = ea;
  g.w = static_cast<const uint8_t *>(w);
  g.l = l;
  g.c = c;
  g.M = M;
  g.N = N;
  g.ksteps = p.ksteps;
  g.ktiles = p.k_pad / BK;
  g.mtiles = p.mtiles;
  g.ntiles = p.ntiles;
  const int grid = (p.ntiles + 7) / 8 * 8 * p.mtiles;
  if (p.nw == 8) {
    if (p.mb == 2) hipLaunchKernelGGL((k_q8_gemm<2, 8>), dim3(grid), dim3(512), 0, s, g);
    else hipLaunchKernelGGL((k_q8_gemm<1, 8>), dim3(grid), dim3(512), 0, s, g);
  } else {
    if (p.mb == 2) hipLaunchKernelGGL((k_q8_gemm<2, 4>), dim3(grid), dim3(256), 0, s, g);
    else hipLaunchKernelGGL((k_q8_gemm<1, 4>), dim3(grid), dim3(256), 0, s, g);
  }
  hip_check(hipGetLastError(), "q8 gemm launch");
}

}  // namespace qnn
