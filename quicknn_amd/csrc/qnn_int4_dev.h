// qnn_int4_dev.h -- device building blocks of the native INT4 matvec kernels
// (qnn_int4.hip: dense projections; qnn_moe.hip: routed experts).
//
// Format (src/core/QuickNN.Quantization.Int4.pas:10-94): per 32 weights an
// fp32 scale s then 16 bytes of offset-binary nibbles n (element j in byte j/2,
// low nibble for even j); value = fl32((n-8)*s).
//
// Device layout (I4Layout): a row is spread over L lanes ("lanes per row",
// a power of two <= 16) and a 64-lane block holds R = 64/L rows.  Lane
// l = r*L + j of block b carries groups j, j+L, j+2L, ... of row b*R + r; its
// step-s group (group s*L + j) sits at
//     nibbles: 16 B at ((b*S + s)*64 + l)               S = ceil(groups / L)
//     scale:    4 B at ((b*Q + s/4)*64 + l)*4 + s%4       Q = ceil(S / 4)
// so every step of a wave is one 16-byte load per lane over 1 KiB of
// contiguous nibbles, and every 4 steps one more over 1 KiB of scales (a
// lane's 4 scales side by side).  Padding groups/rows hold scale 0.
//
// A wave computes the rows of one block ("tile") over a K-range of steps; the
// L partial sums of a row meet by cross-lane reduction.  The activation slice
// of a workgroup is staged in LDS as 16-bit fixed point per 32-group (two int8
// planes); the inner product runs on the raw nibble bytes with v_dot4_i32_i8
// and folds the offset and both scales once per group:
//     sum_j (n_j - 8) s x_j ~= s * s2 * (sum_j n_j (256 q1_j + q2_j) - 8 sum_j (256 q1_j + q2_j))
// (exact integer arithmetic inside a group; fp32 across groups; relative
// error of the activation representation <= 2^-16 of the group's max|x|).
//
// Loads go through buffer resources (reads past the end return 0) and are
// issued without per-lane branches (out-of-range steps and tokens re-read a
// valid address and are masked when staged; only whole passes beyond the
// slice are skipped, on a uniform condition), so the compiler can wait for
// the activation loads alone while the weight loads are still in flight.
#pragma once
#include "qnn_exchange.h"

namespace qnn {
namespace dev {

__device__ __forceinline__ float silu(float g) {
  // Clamped SiLU of moe.comp:118 / QwenHybrid.CPU.pas:242-246.
  return g >= 20.0f ? g : (g <= -20.0f ? 0.0f : g / (1.0f + expf(-g)));
}

__device__ __forceinline__ uint32_t sel4u(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Wave index as a scalar (uniform) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Activation planes of a K-slice in (dynamic) LDS: per token and group, 8
// words of the high int8 plane and 8 of the low plane, padded to 80 bytes (an
// odd number of 16-byte quads: the 16 lanes of a row read 16 consecutive
// groups, whose 16-byte pieces then fall in distinct bank quads), s2 and
// -8*sum(256 q1 + q2).
struct XPlanes {
  uint32_t *q;  // [tokens][groups][kXWords]: words 0-7 high plane, 8-15 low plane, 16-19 padding
  float *s2;    // [tokens][groups]
  int *off;     // [tokens][groups]
  int groups;   // groups per token in the slice
};
constexpr int kXWords = 20;  // words per (token, group): 8 high + 8 low + 4 padding

__host__ __device__ constexpr size_t xplanes_bytes(int tokens, int groups) {
  return size_t(tokens) * groups * (kXWords * 4 + 8);
}
__device__ __forceinline__ XPlanes xplanes_at(void *lds, int tokens, int groups) {
  XPlanes p;
  p.q = static_cast<uint32_t *>(lds);
  p.s2 = reinterpret_cast<float *>(p.q + size_t(tokens) * groups * kXWords);
  p.off = reinterpret_cast<int *>(p.s2 + size_t(tokens) * groups);
  p.groups = groups;
  return p;
}

// float4 loads per thread and token covering a slice of GSW steps at up to 16
// lanes per row.
template <int GSW>
constexpr int x_iters() { return (GSW * 16 * 32 + 1023) / 1024; }

// Raw buffer resource over `bytes` bytes at `base` (gfx9 raw-buffer word 3):
// loads at offsets >= bytes return 0 instead of touching memory, and the
// per-step offsets of a load sequence travel in scalar registers.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc rsrc(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(uint32_t(min(bytes, size_t(0xFFFFFFFFu)))),
                                           0x00020000);
}
// Resources that end with block b's weights (its nibbles, its scale pieces),
// so a wave's steps past the block's last step read zeros rather than the
// next block's bytes (a K-slice longer than the steps left in the block).
__device__ __forceinline__ Rsrc block_nib_rsrc(const void *nib, const I4Layout &l, int b) {
  return rsrc(nib, size_t(b + 1) * l.steps * 1024);
}
__device__ __forceinline__ Rsrc block_scl_rsrc(const void *scl, const I4Layout &l, int b) {
  return rsrc(scl, size_t(b + 1) * l.quads() * 1024);
}
// AUX = 16 sets SC1: the load is coherent at device (agent) scope, for data
// another XCD wrote inside the same launch.
template <int AUX = 0>
__device__ __forceinline__ uint4 ld128(Rsrc r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, int(voff), int(soff), AUX);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
constexpr int kCoherent = 16;
// AUX = 2 sets NT: a streaming (non-temporal) load.  Weight bytes are read
// once per launch, so they stream and leave the L2 to the activation slices
// and the split-K exchange (measured: Qwen3-4B decode MLP 16.3 -> 15.9 us,
// 6144 x 2048 matvec 6.1 -> 5.8 us).
constexpr int kStream = 2;
__device__ __forceinline__ float ld32f(Rsrc r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, int(voff), int(soff), 0));
}

// Loads the 4-float pieces of elements [e0, ...) of MT activation rows, one
// per thread per pass; row m starts at byte rowoff(m) of buffer xr_src (rows
// hold a multiple of 4 floats, 16-byte aligned).  Nothing is masked here, so
// no load waits for another; stage_x zeroes the pieces outside the slice, the
// row or the token count.
// `ne` (uniform) bounds the passes to those the slice needs.
template <int MT, int GSW, int AUX = 0, class OffF>
__device__ __forceinline__ void load_x(float4 (&xr)[MT][x_iters<GSW>()], Rsrc src, OffF rowoff, int mt, int e0,
                                       int ne, int tid) {
  const int passes = (ne + 1023) >> 10;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint32_t base = rowoff(m < mt ? m : 0) + uint32_t(e0 + tid * 4) * 4u;
#pragma unroll
    for (int it = 0; it < x_iters<GSW>(); ++it) {
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (it < passes) {
        const uint4 v = ld128<AUX>(src, base, uint32_t(it) * 4096u);
        f = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
      }
      xr[m][it] = f;
    }
  }
}

// This wave's weight stream for GSW steps from step s0 of block b (lane wl of
// the block): nibble pieces and scales.  Steps at or past the matrix's last
// step read other blocks or zeros (masked in dot).
// Scale pieces a GSW-step window needs: windows start at a multiple of their
// (power-of-two) length, so steps s0..s0+GSW-1 lie in GSW/4 pieces, or in one
// piece at offset s0 % 4 when GSW <= 2.
template <int GSW>
constexpr int scale_quads() { return GSW >= 4 ? GSW / 4 : 1; }
template <int GSW>
__device__ __forceinline__ void pick_scales(float (&sc)[GSW], const uint4 (&q)[scale_quads<GSW>()], int s0) {
  if constexpr (GSW >= 4) {
#pragma unroll
    for (int g = 0; g < GSW; ++g) sc[g] = __uint_as_float(sel4u(q[g >> 2], g & 3));
  } else {
    const int o = s0 & 3;
#pragma unroll
    for (int g = 0; g < GSW; ++g) sc[g] = __uint_as_float(sel4u(q[0], (o + g) & 3));
  }
}
// nib_off / scl_off: per-lane byte offsets of the lane's matrix within the
// resources (lets lanes of one wave read two matrices through one uniform
// resource instead of a divergent one).
// load_wq issues the loads only; pick_scales(sc, q, s0) then selects the
// scales (for GSW < 4 a data-dependent select that waits for the scale load,
// so callers that issue more loads do so before it).
template <int GSW>
__device__ __forceinline__ void load_wq(uint4 (&w)[GSW], uint4 (&q)[scale_quads<GSW>()], Rsrc nib, Rsrc scl,
                                        const I4Layout &l, int b, int s0, int wl, uint32_t nib_off = 0,
                                        uint32_t scl_off = 0) {
  const uint32_t at = uint32_t((size_t(b) * l.steps + s0) * 64 + wl);
  const uint32_t qat = uint32_t((size_t(b) * l.quads() + (s0 >> 2)) * 64 + wl);
#pragma unroll
  for (int i = 0; i < scale_quads<GSW>(); ++i) q[i] = ld128<kStream>(scl, scl_off + qat * 16u, uint32_t(i) * 1024u);
#pragma unroll
  for (int g = 0; g < GSW; ++g) w[g] = ld128<kStream>(nib, nib_off + at * 16u, uint32_t(g) * 1024u);
}
template <int GSW>
__device__ __forceinline__ void load_w(uint4 (&w)[GSW], float (&sc)[GSW], Rsrc nib, Rsrc scl, const I4Layout &l, int b,
                                       int s0, int wl, uint32_t nib_off = 0, uint32_t scl_off = 0) {
  uint4 q[scale_quads<GSW>()];
  load_wq<GSW>(w, q, nib, scl, l, b, s0, wl, nib_off, scl_off);
  pick_scales<GSW>(sc, q, s0);
}

// Quantises the loaded slice per 32-element group to 16-bit fixed point,
// x ~= s2 * (256*q1 + q2) with q1, q2 in [-127, 127]:
//   s1 = amax/127, q1 = rint(x/s1), r = x - q1*s1, s2 = s1/256, q2 = rint(r/s2)
// (|x - s2(256 q1 + q2)| <= s2/2 = amax/65024, up to s2 where the clamp of
// q2 to 127 bites).  1/s1 is the hardware reciprocal, and the rounding is
// fma(v, 1/s, 1.5 * 2^23): the sum rounds v/s to the nearest integer (ties
// to even) inside the float, whose low mantissa bits then hold it in two's
// complement, so byte 0 of the float's bits is the int8 and the float minus
// 1.5 * 2^23 is the exact q as a float.  Every kernel stages through these
// helpers, so all paths see the same planes.
// The int8 planes match the nibble bytes of a weight dword: dword c of a group
// holds elements 8c..8c+7, its low nibbles are the even elements and its high
// nibbles the odd ones, so plane word 2c packs x[8c+0,2,4,6] and word 2c+1
// x[8c+1,3,5,7].  Words 0-7 of an entry are the high plane, 8-15 the low plane.
// Pieces of token m >= mt, of element >= ne within the slice or of row
// element >= k are zero (e0 = first element of the slice).
constexpr float kRound = 12582912.0f;      // 1.5 * 2^23
constexpr uint32_t kRoundBits = 0x4B400000u;  // its bits
struct GroupScale {
  float s1, inv, inv2;
};
__device__ __forceinline__ GroupScale group_scale(float amax) {
  GroupScale g;
  g.s1 = amax * (1.0f / 127.0f);
  g.inv = g.s1 > 1e-30f ? __builtin_amdgcn_rcpf(g.s1) : 0.0f;  // groups below 1e-28 stage as zeros
  g.inv2 = g.inv * 256.0f;
  return g;
}
// One element: the rounded floats whose bits carry q1 (b1) and q2 (b2).
__device__ __forceinline__ void quant_elem(float x, const GroupScale &g, uint32_t &b1, uint32_t &b2) {
  const float f1 = fmaf(x, g.inv, kRound);
  const float r = fmaf(kRound - f1, g.s1, x);  // x - q1 * s1
  const float f2 = __builtin_amdgcn_fmed3f(fmaf(r, g.inv2, kRound), kRound - 127.0f, kRound + 127.0f);
  b1 = __float_as_uint(f1);
  b2 = __float_as_uint(f2);
}
// sum(256 q1 + q2) over N elements from their bits (exact: the true sum is small).
template <int N>
__device__ __forceinline__ int quant_sum(const uint32_t (&b1)[N], const uint32_t (&b2)[N]) {
  uint32_t s1 = 0, s2 = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    s1 += b1[i];
    s2 += b2[i];
  }
  return int((s1 << 8) + s2 - uint32_t(N) * 257u * kRoundBits);
}
// Byte 0 of a and of b -> bytes 0 and 1 (bytes 2, 3 zero).
__device__ __forceinline__ uint32_t pack2(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x0C0C0400u); }
// The low halves of a and b -> one word.
__device__ __forceinline__ uint32_t join2(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }

// Cross-lane reductions over aligned groups of 4 or 8 lanes (DPP, within a
// 16-lane row): quad swaps of 1 and 2, then the other half of 8.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float max_lanes4(float v) {
  v = fmaxf(v, __uint_as_float(dpp<0xB1>(__float_as_uint(v))));  // quad_perm [1,0,3,2]
  return fmaxf(v, __uint_as_float(dpp<0x4E>(__float_as_uint(v))));  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ float max_lanes8(float v) {
  v = max_lanes4(v);
  return fmaxf(v, __uint_as_float(dpp<0x141>(__float_as_uint(v))));  // row_half_mirror
}
__device__ __forceinline__ int sum_lanes4(int v) {
  v += int(dpp<0xB1>(uint32_t(v)));
  return v + int(dpp<0x4E>(uint32_t(v)));
}
__device__ __forceinline__ int sum_lanes8(int v) {
  v = sum_lanes4(v);
  return v + int(dpp<0x141>(uint32_t(v)));
}

// One 4-element piece: elements e..e+3 (within the slice) of token m; the 8
// lanes of a 32-group meet through DPP, so every lane of the wave runs it.
__device__ __forceinline__ void stage_piece(const XPlanes &xs, const float4 v, int m, int e, int lane) {
  const float amax = max_lanes8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  const GroupScale gs = group_scale(amax);
  uint32_t b1[4], b2[4];
  quant_elem(v.x, gs, b1[0], b2[0]);
  quant_elem(v.y, gs, b1[1], b2[1]);
  quant_elem(v.z, gs, b1[2], b2[2]);
  quant_elem(v.w, gs, b1[3], b2[3]);
  const int sumq = sum_lanes8(quant_sum<4>(b1, b2));
  const int g = e >> 5;
  if (g < xs.groups) {
    const int i0 = e & 31;  // element 8c + (i0 & 7) of group g
    const int c = i0 >> 3, half = (i0 >> 2) & 1;
    const size_t mg = size_t(m) * xs.groups + g;
    uint16_t *ph = reinterpret_cast<uint16_t *>(xs.q + mg * kXWords);
    uint16_t *pl = ph + 16;
    // bytes for even slots (elements +0, +2) and odd slots (+1, +3) of this half dword
    ph[(2 * c) * 2 + half] = uint16_t(pack2(b1[0], b1[2]));
    ph[(2 * c + 1) * 2 + half] = uint16_t(pack2(b1[1], b1[3]));
    pl[(2 * c) * 2 + half] = uint16_t(pack2(b2[0], b2[2]));
    pl[(2 * c + 1) * 2 + half] = uint16_t(pack2(b2[1], b2[3]));
    if ((lane & 7) == 0) {
      xs.s2[mg] = gs.s1 * 0.00390625f;
      xs.off[mg] = -8 * sumq;
    }
  }
}

template <int MT, int GSW>
__device__ __forceinline__ void stage_x(const XPlanes &xs, const float4 (&xr)[MT][x_iters<GSW>()], int mt, int e0,
                                        int ne, int k, int tid, int lane) {
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int it = 0; it < x_iters<GSW>(); ++it) {
      if (it * 1024 >= ne) break;  // uniform: passes past the slice
      const int e = (it * 256 + tid) * 4;  // first element of this thread, within the slice
      const bool ok = m < mt && e < ne && e0 + e < k;
      stage_piece(xs, ok ? xr[m][it] : make_float4(0.f, 0.f, 0.f, 0.f), m, e, lane);
    }
  }
}

// Planes of one (token, group) dword from 8 elements held by this lane; the
// 4 lanes of the group (aligned, adjacent) meet through DPP.  For the
// matrix-core dot, which multiplies signed nibbles scaled by 16 (dot_mf), the
// entry holds s2/16 and no offset.
__device__ __forceinline__ void stage_dword(const XPlanes &xs, const float (&v)[8], int m, int g, int c) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const GroupScale gs = group_scale(max_lanes4(amax));
  uint32_t b1[8], b2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) quant_elem(v[i], gs, b1[i], b2[i]);
  if (g < xs.groups) {
    const size_t mg = size_t(m) * xs.groups + g;
    uint2 *pq = reinterpret_cast<uint2 *>(xs.q + mg * kXWords);
    pq[c] = make_uint2(join2(pack2(b1[0], b1[2]), pack2(b1[4], b1[6])), join2(pack2(b1[1], b1[3]), pack2(b1[5], b1[7])));
    pq[4 + c] =
        make_uint2(join2(pack2(b2[0], b2[2]), pack2(b2[4], b2[6])), join2(pack2(b2[1], b2[3]), pack2(b2[5], b2[7])));
    if (c == 0) xs.s2[mg] = gs.s1 * (0.00390625f * 0.0625f);
  }
}

// Slices of at most 512 elements, MT a multiple of 4: in pass p wave w stages
// token 4p + w, lane l elements 8l..8l+7 of the slice (dword l%4 of group
// l/4), so no thread idles and a lane writes whole plane words.  The planes
// are those stage_x writes.
template <int MT, class OffF>
__device__ __forceinline__ void load_x_quads(float4 (&xr)[MT / 4][2], Rsrc src, OffF rowoff, int mt, int e0, int wave,
                                             int lane) {
#pragma unroll
  for (int p = 0; p < MT / 4; ++p) {
    const int m = 4 * p + wave;
    const uint32_t base = rowoff(m < mt ? m : 0) + uint32_t(e0 + lane * 8) * 4u;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint4 v = ld128(src, base, uint32_t(h) * 16u);
      xr[p][h] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    }
  }
}
template <int MT>
__device__ __forceinline__ void stage_x_quads(const XPlanes &xs, const float4 (&xr)[MT / 4][2], int mt, int e0, int ne,
                                              int k, int wave, int lane) {
#pragma unroll
  for (int p = 0; p < MT / 4; ++p) {
    const int m = 4 * p + wave, e = lane * 8;
    float v[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool ok = m < mt && e + 4 * h < ne && e0 + e + 4 * h < k;
      const float4 f = ok ? xr[p][h] : make_float4(0.f, 0.f, 0.f, 0.f);
      v[4 * h] = f.x;
      v[4 * h + 1] = f.y;
      v[4 * h + 2] = f.z;
      v[4 * h + 3] = f.w;
    }
    stage_dword(xs, v, m, lane >> 2, lane & 3);
  }
}

// Dequantise-free integer dot over this lane's groups (steps 0..ns-1 of the
// slice; group s*L + j of the slice for lane j of its row):
//   isum = 256 * dot(n, q1) + dot(n, q2) - 8 * sum(256 q1 + q2)  (exact, < 2^24)
//   acc += float(isum) * (s * s2).
template <int MT, int GSW>
__device__ __forceinline__ void dot(float (&acc)[MT], const uint4 (&w)[GSW], const float (&sc)[GSW],
                                    const XPlanes &xs, int lanes, int j, int ns) {
#pragma unroll
  for (int g = 0; g < GSW; ++g) {
    if (g < ns) {
      const int gl = g * lanes + j;
      uint32_t nlo[4], nhi[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t wd = sel4u(w[g], c);
        nlo[c] = wd & 0x0F0F0F0Fu;
        nhi[c] = (wd >> 4) & 0x0F0F0F0Fu;
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const size_t mg = size_t(m) * xs.groups + gl;
        const uint4 *q = reinterpret_cast<const uint4 *>(xs.q + mg * kXWords);
        const uint4 h0 = q[0], h1 = q[1], l0 = q[2], l1 = q[3];
        int ah0 = 0, ah1 = 0, al0 = 0, al1 = 0;
        ah0 = __builtin_amdgcn_sdot4(int(nlo[0]), int(h0.x), ah0, false);
        ah1 = __builtin_amdgcn_sdot4(int(nhi[0]), int(h0.y), ah1, false);
        al0 = __builtin_amdgcn_sdot4(int(nlo[0]), int(l0.x), al0, false);
        al1 = __builtin_amdgcn_sdot4(int(nhi[0]), int(l0.y), al1, false);
        ah0 = __builtin_amdgcn_sdot4(int(nlo[1]), int(h0.z), ah0, false);
        ah1 = __builtin_amdgcn_sdot4(int(nhi[1]), int(h0.w), ah1, false);
        al0 = __builtin_amdgcn_sdot4(int(nlo[1]), int(l0.z), al0, false);
        al1 = __builtin_amdgcn_sdot4(int(nhi[1]), int(l0.w), al1, false);
        ah0 = __builtin_amdgcn_sdot4(int(nlo[2]), int(h1.x), ah0, false);
        ah1 = __builtin_amdgcn_sdot4(int(nhi[2]), int(h1.y), ah1, false);
        al0 = __builtin_amdgcn_sdot4(int(nlo[2]), int(l1.x), al0, false);
        al1 = __builtin_amdgcn_sdot4(int(nhi[2]), int(l1.y), al1, false);
        ah0 = __builtin_amdgcn_sdot4(int(nlo[3]), int(h1.z), ah0, false);
        ah1 = __builtin_amdgcn_sdot4(int(nhi[3]), int(h1.w), ah1, false);
        al0 = __builtin_amdgcn_sdot4(int(nlo[3]), int(l1.z), al0, false);
        al1 = __builtin_amdgcn_sdot4(int(nhi[3]), int(l1.w), al1, false);
        const int isum = ((ah0 + ah1) << 8) + (al0 + al1) + xs.off[mg];
        acc[m] = fmaf(float(isum), sc[g] * xs.s2[mg], acc[m]);
      }
    }
  }
}

// ---- Several tokens on the int8 matrix cores (L = 1, MT >= 4, GSW >= 4).
// Per group and 16-row quarter rq of the block, with 9-16 tokens one
// v_mfma_i32_16x16x32_i8 per activation plane (up to 8 tokens: one for both,
// below): A = the plane (16 tokens x 32 elements; lane l gives
// token l%16, elements 8c..8c+7 of the group, c = l/16, as plane words 2c and
// 2c+1), B = the weights (32 elements x 16 rows; lane l gives row 16rq + l%16,
// the same elements: the low then the high nibbles of its dword c) as the
// signed bytes 16 (n - 8): after n ^ 8 a nibble read as signed 4 bits is
// n - 8, and with the nibble in the high half of its byte the byte is 16 (n -
// 8), so the -8 needs no offset term and no masking of signs.  Both orders
// are [8c+0,2,4,6, 8c+1,3,5,7], so 256 D_high + D_low is 16 times the group's
// exact sum 256 dot(n, q1) + dot(n, q2) - 8 sum(256 q1 + q2) that dot()
// forms with v_dot4 (an integer below 2^28 with four zero low bits, so its
// float is exact and 16 times dot()'s), and the planes hold s2 / 16, so
// s * s2 / 16 is dot()'s scale product over 16 exactly: the fma gives the
// same float, and results are bit-identical to dot() (while s * s2 / 16 stays
// a normal float).  Lane l holds D[4c + r][l%16], r = 0..3: tokens 4c..4c+3
// of row 16rq + l%16.  Token rows >= MT read token 0's plane and are
// discarded.
//
// The weights arrive as the layout stores them, lane l holding row l's 16
// bytes of each step (one 16-byte load per lane and step: 4-byte loads in that
// pattern streamed 30% slower), and are put in that pattern at use: dword c of
// row 16rq + l%16 is a 4 x 4 transpose across the four 16-lane rows (two
// 32-lane and two 16-lane swaps per step).  The scales of those rows come as
// one 16-byte scale piece per quarter and 4 steps.
template <int GSW>
struct MfWeights {
  uint4 w[GSW];        // [step]: row l's 16 bytes
  float sc[GSW][4];    // [step][quarter]: the scale of row 16*quarter + l%16
};
// (dword c of row 16rq + l%16 for rq = 0..3) from (row l's dwords 0..3).
__device__ __forceinline__ void mf_transpose(uint32_t (&o)[4], const uint4 &v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  o[0] = c[0];
  o[1] = c[1];
  o[2] = d[0];
  o[3] = d[1];
}
template <int GSW>
__device__ __forceinline__ void load_w_mf(MfWeights<GSW> &mw, Rsrc nib, Rsrc scl, const I4Layout &l, int b, int s0,
                                          int lane) {
  static_assert(GSW % 4 == 0, "scale pieces hold 4 aligned steps");
  const int p = lane & 15;
  const uint32_t at = uint32_t(size_t(b) * l.steps + s0) * 1024u + uint32_t(lane * 16);
  const uint32_t qat = uint32_t((size_t(b) * l.quads() + (s0 >> 2)) * 64 + p) * 16u;
  uint4 q[GSW / 4][4];
#pragma unroll
  for (int i = 0; i < GSW / 4; ++i)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) q[i][rq] = ld128<kStream>(scl, qat + uint32_t(rq) * 256u, uint32_t(i) * 1024u);
#pragma unroll
  for (int g = 0; g < GSW; ++g) mw.w[g] = ld128<kStream>(nib, at, uint32_t(g) * 1024u);
#pragma unroll
  for (int g = 0; g < GSW; ++g)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) mw.sc[g][rq] = __uint_as_float(sel4u(q[g >> 2][rq], g & 3));
}

typedef int mf_i32x4 __attribute__((ext_vector_type(4)));

// Up to 8 tokens: both planes in one product.  A row p = 2 * token + plane
// (plane 0 the high plane), so lane l holds D[4c + r][l%16] = token 2c + r/2,
// plane r%2: the high and the low sum of tokens 2c and 2c + 1 sit in the
// lane's own result registers.  Each lane finishes 2 (row, token) sums per
// quarter and step instead of 4, with half the products and no lane swaps.
template <int MT>
constexpr int mf_per_lane() { return MT <= 8 ? 2 : 4; }
template <int MT>
__device__ __forceinline__ int mf_token(int lane, int r) {
  if constexpr (MT <= 8)
    return 2 * (lane >> 4) + r;
  else
    return 4 * (lane >> 4) + r;
}

// acc[rq][r] += the group sums of steps 0..ns-1 for token mf_token(lane, r),
// row 16rq + l%16 (the layouts above), in step order.
template <int MT, int GSW>
__device__ __forceinline__ void dot_mf(float (&acc)[4][mf_per_lane<MT>()], const MfWeights<GSW> &mw,
                                       const XPlanes &xs, int ns, int lane) {
  constexpr int R = mf_per_lane<MT>();
  const int p = lane & 15, c = lane >> 4;
  const int tp = MT <= 8 ? (p >> 1) : p;  // A row token
  const int ta = tp < MT ? tp : 0;
  const int aw = MT <= 8 ? 8 * (p & 1) + 2 * c : 2 * c;  // A words within the entry
  int tk[R];
#pragma unroll
  for (int r = 0; r < R; ++r) tk[r] = mf_token<MT>(lane, r) < MT ? mf_token<MT>(lane, r) : 0;
#pragma unroll
  for (int g = 0; g < GSW; ++g) {
    if (g < ns) {
      const uint32_t *qa = xs.q + (size_t(ta) * xs.groups + g) * kXWords;
      const long ah = *reinterpret_cast<const long *>(qa + aw);
      float s2[R];
#pragma unroll
      for (int r = 0; r < R; ++r) s2[r] = xs.s2[size_t(tk[r]) * xs.groups + g];
      uint32_t wq[4];
      const uint4 ws = make_uint4(mw.w[g].x ^ 0x88888888u, mw.w[g].y ^ 0x88888888u, mw.w[g].z ^ 0x88888888u,
                                  mw.w[g].w ^ 0x88888888u);  // nibbles n ^ 8: n - 8 as signed nibbles
      mf_transpose(wq, ws);
      // Up to 8 tokens: the step's four products first, so that each one's
      // latency is covered by the others before its swaps read it.
      mf_i32x4 d4[MT <= 8 ? 4 : 1];
      if constexpr (MT <= 8) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const uint32_t wd = wq[rq];
          const long bw = long((wd << 4) & 0xF0F0F0F0u) | (long(wd & 0xF0F0F0F0u) << 32);  // 16 (n - 8)
          const mf_i32x4 z = {0, 0, 0, 0};
          d4[rq] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, bw, z, 0, 0, 0);
        }
      }
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const uint32_t wd = wq[rq];
        const long bw = long((wd << 4) & 0xF0F0F0F0u) | (long(wd & 0xF0F0F0F0u) << 32);  // 16 (n - 8)
        const mf_i32x4 z = {0, 0, 0, 0};
        int hi[R], lo[R];
        if constexpr (MT <= 8) {
          const mf_i32x4 dh = d4[rq];
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            hi[r] = dh[2 * r];
            lo[r] = dh[2 * r + 1];
          }
        } else {
          const mf_i32x4 dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, bw, z, 0, 0, 0);
          const long al = *reinterpret_cast<const long *>(qa + 8 + 2 * c);
          const mf_i32x4 dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, bw, z, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            hi[r] = dh[r];
            lo[r] = dl[r];
          }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int isum16 = (hi[r] << 8) + lo[r];  // 16 x the exact group sum
          acc[rq][r] = fmaf(float(isum16), mw.sc[g][rq] * s2[r], acc[rq][r]);
        }
      }
    }
  }
}

// The MFMA layout -> one row per lane (acc[m] = token m of row `lane`),
// through this wave's [MT][64] LDS slot.
template <int MT>
__device__ __forceinline__ void mf_to_rows(float (&acc)[MT], const float (&accm)[4][mf_per_lane<MT>()], float *slot,
                                           int lane) {
  const int p = lane & 15;
#pragma unroll
  for (int rq = 0; rq < 4; ++rq)
#pragma unroll
    for (int r = 0; r < mf_per_lane<MT>(); ++r)
      if (mf_token<MT>(lane, r) < MT) slot[mf_token<MT>(lane, r) * 64 + 16 * rq + p] = accm[rq][r];
  wave_lds_sync();
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = slot[m * 64 + lane];
}

// Sum over the L lanes of each row (L a power of two): afterwards every lane
// of a row holds the row total.  Pairwise order, identical in every launch.
template <int MT>
__device__ __forceinline__ void reduce_lanes(float (&acc)[MT], int lanes) {
  for (int o = 1; o < lanes; o <<= 1) {
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] += __shfl_xor(acc[m], o);
  }
}

}  // namespace dev
}  // namespace qnn
