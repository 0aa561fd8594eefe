// qnn_int4_dev.h -- device building blocks of the native INT4 matvec kernels
// (qnn_int4.hip: dense projections; qnn_moe.hip: routed experts).
//
// Format (src/core/QuickNN.Quantization.Int4.pas:10-94): per 32 weights an
// fp32 scale s then 16 bytes of offset-binary nibbles n (element j in byte j/2,
// low nibble for even j); value = fl32((n-8)*s).  Device layout: I4Layout.
//
// A workgroup is 4 wavefronts on one 64-row tile (one row per lane) and a
// K-slice of GS = 4*GSW groups; wave w streams groups [w*GSW, (w+1)*GSW).
// Every weight load is a 16-byte global_load_dwordx4 and consecutive lanes
// read consecutive 16-byte pieces.  The activation slice is staged in LDS as
// 16-bit fixed point per 32-group (two int8 planes); the inner product runs on
// the raw nibble bytes with v_dot4_i32_i8 and folds the offset and both scales
// once per group:
//     sum_j (n_j - 8) s x_j ~= s * s2 * (sum_j n_j (256 q1_j + q2_j) - 8 sum_j (256 q1_j + q2_j))
// (exact integer arithmetic inside a group; fp32 across groups; relative
// error of the activation representation <= 2^-16 of the group's max|x|).
#pragma once
#include "qnn_internal.h"

namespace qnn {
namespace dev {

__device__ __forceinline__ float silu(float g) {
  // Clamped SiLU of moe.comp:118 / QwenHybrid.CPU.pas:242-246.
  return g >= 20.0f ? g : (g <= -20.0f ? 0.0f : g / (1.0f + expf(-g)));
}

__device__ __forceinline__ uint32_t sel4u(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Hardware XCC id of the executing wave (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() { return int(__builtin_amdgcn_s_getreg((3 << 11) | 20)) & 15; }

// Activation rows staged for one K-slice: per token and group, 8 words of the
// high int8 plane, 8 of the low plane, s2 and -8*sum(256 q1 + q2).
template <int MT, int GS>
struct XTile {
  uint32_t h[MT][GS][8];
  uint32_t l[MT][GS][8];
  float s2[MT][GS];
  int off[MT][GS];
};

template <int GS>
constexpr int x_iters() { return (GS * 32 + 1023) / 1024; }

// Loads elements [g0*32, g0*32 + ng*32) of MT activation rows, 4 per thread per
// pass; row(m) returns the row's base or nullptr (token absent: zeros).
template <int MT, int GS, class RowF>
__device__ __forceinline__ void load_x(float4 (&xr)[MT][x_iters<GS>()], RowF row, int g0, int ng, int k, bool vec4,
                                       int tid) {
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float *xp = row(m);
#pragma unroll
    for (int it = 0; it < x_iters<GS>(); ++it) {
      const int e = (it * 256 + tid) * 4;
      const int kk = g0 * 32 + e;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (xp != nullptr && e < ng * 32) {
        if (kk + 3 < k && vec4) {
          v = *reinterpret_cast<const float4 *>(xp + kk);
        } else if (kk + 3 < k) {
          v.x = xp[kk]; v.y = xp[kk + 1]; v.z = xp[kk + 2]; v.w = xp[kk + 3];
        } else {
          if (kk < k) v.x = xp[kk];
          if (kk + 1 < k) v.y = xp[kk + 1];
          if (kk + 2 < k) v.z = xp[kk + 2];
        }
      }
      xr[m][it] = v;
    }
  }
}

// This wave's weight stream: GSW scales then GSW nibble pieces, in group
// order (loads return in issue order, so group g is usable once it lands).
// nib/sclf point at the wave's first group gq0 of row srow of the stored tile.
template <int GSW>
__device__ __forceinline__ void load_w(uint4 (&w)[GSW], float (&sc)[GSW], const uint4 *nib, const float *sclf,
                                       int gq0, int ngw) {
  if (GSW >= 4) {  // whole scale quads: one 16-byte load per 4 groups
#pragma unroll
    for (int q = 0; q < GSW / 4; ++q)
      if (4 * q < ngw) {
        const float4 s4 = *reinterpret_cast<const float4 *>(sclf + q * 256);
        sc[4 * q] = s4.x;
        sc[4 * q + 1] = s4.y;
        sc[4 * q + 2] = s4.z;
        sc[4 * q + 3] = s4.w;
      }
  } else {
#pragma unroll
    for (int g = 0; g < GSW; ++g) {
      if (g < ngw) {
        const int gg = gq0 + g;  // scale of group gg: quad gg/4, component gg%4
        sc[g] = sclf[((gg >> 2) - (gq0 >> 2)) * 256 + (gg & 3)];
      }
    }
  }
#pragma unroll
  for (int g = 0; g < GSW; ++g)
    if (g < ngw) w[g] = nib[g * 64];
}

// Quantises the loaded slice per 32-element group to 16-bit fixed point,
// x ~= s2 * (256*q1 + q2) with q1, q2 in [-127, 127]:
//   s1 = amax/127, q1 = rint(x/s1), r = x - q1*s1, s2 = s1/256, q2 = rint(r/s2)
// (|x - s2(256 q1 + q2)| <= s2/2 = amax/65024).  The int8 planes match the
// nibble bytes of a weight dword: dword c of a group holds elements 8c..8c+7,
// its low nibbles are the even elements and its high nibbles the odd ones, so
// word 2c packs x[8c+0,2,4,6] and word 2c+1 x[8c+1,3,5,7].
template <int MT, int GS>
__device__ __forceinline__ void stage_x(XTile<MT, GS> &xs, const float4 (&xr)[MT][x_iters<GS>()], int tid, int lane) {
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int it = 0; it < x_iters<GS>(); ++it) {
      const int e = (it * 256 + tid) * 4;  // first element of this thread, within the slice
      const float4 v = xr[m][it];
      float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      amax = fmaxf(amax, __shfl_xor(amax, 4));
      const float s1 = amax / 127.0f;
      const float inv = s1 > 0.0f ? 1.0f / s1 : 0.0f;
      const float inv2 = inv * 256.0f;
      int h[4], l[4];
      const float xv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float q1 = fminf(127.0f, fmaxf(-127.0f, rintf(xv[j] * inv)));
        const float r = fmaf(-q1, s1, xv[j]);
        const float q2 = fminf(127.0f, fmaxf(-127.0f, rintf(r * inv2)));
        h[j] = int(q1);
        l[j] = int(q2);
      }
      int sumq = (256 * h[0] + l[0]) + (256 * h[1] + l[1]) + (256 * h[2] + l[2]) + (256 * h[3] + l[3]);
      sumq += __shfl_xor(sumq, 1);
      sumq += __shfl_xor(sumq, 2);
      sumq += __shfl_xor(sumq, 4);
      if (e < GS * 32) {
        const int g = e >> 5, i0 = e & 31;  // element 8c + (i0 & 7) of group g
        const int c = i0 >> 3, half = (i0 >> 2) & 1;
        // bytes for even slots (elements +0, +2) and odd slots (+1, +3) of this half dword
        const uint32_t he = (uint32_t(h[0]) & 255u) | ((uint32_t(h[2]) & 255u) << 8);
        const uint32_t ho = (uint32_t(h[1]) & 255u) | ((uint32_t(h[3]) & 255u) << 8);
        const uint32_t le = (uint32_t(l[0]) & 255u) | ((uint32_t(l[2]) & 255u) << 8);
        const uint32_t lo = (uint32_t(l[1]) & 255u) | ((uint32_t(l[3]) & 255u) << 8);
        uint16_t *ph = reinterpret_cast<uint16_t *>(&xs.h[m][g][0]);
        uint16_t *pl = reinterpret_cast<uint16_t *>(&xs.l[m][g][0]);
        ph[(2 * c) * 2 + half] = uint16_t(he);
        ph[(2 * c + 1) * 2 + half] = uint16_t(ho);
        pl[(2 * c) * 2 + half] = uint16_t(le);
        pl[(2 * c + 1) * 2 + half] = uint16_t(lo);
        if ((lane & 7) == 0) {
          xs.s2[m][g] = s1 * 0.00390625f;
          xs.off[m][g] = -8 * sumq;
        }
      }
    }
  }
}

// Dequantise-free integer dot over this wave's groups, per group and token:
//   isum = 256 * dot(n, q1) + dot(n, q2) - 8 * sum(256 q1 + q2)  (exact, < 2^24)
//   acc += float(isum) * (s * s2).
template <int MT, int GS, int GSW>
__device__ __forceinline__ void dot(float (&acc)[MT], const uint4 (&w)[GSW], const float (&sc)[GSW],
                                    const XTile<MT, GS> &xs, int gw0, int ngw) {
#pragma unroll
  for (int g = 0; g < GSW; ++g) {
    if (g < ngw) {
      const int gl = gw0 + g;
      uint32_t nlo[4], nhi[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t wd = sel4u(w[g], c);
        nlo[c] = wd & 0x0F0F0F0Fu;
        nhi[c] = (wd >> 4) & 0x0F0F0F0Fu;
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const uint4 *qh = reinterpret_cast<const uint4 *>(&xs.h[m][gl][0]);
        const uint4 *ql = reinterpret_cast<const uint4 *>(&xs.l[m][gl][0]);
        const uint4 h0 = qh[0], h1 = qh[1], l0 = ql[0], l1 = ql[1];
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
        const int isum = ((ah0 + ah1) << 8) + (al0 + al1) + xs.off[m][gl];
        acc[m] = fmaf(float(isum), sc[g] * xs.s2[m][gl], acc[m]);
      }
    }
  }
}

// ---- split-K exchange between workgroups of one tile --------------------
// With `local` set, every workgroup of the tile runs on one XCD and the data
// meet in that XCD's L2 through plain stores/loads; otherwise they travel as
// device-scope atomic stores/loads, which are coherent across XCDs by
// themselves (a device-scope fence would write back and invalidate the whole
// L2).  The writer waits for its stores to complete before taking a ticket.
__device__ __forceinline__ void xstore(float *p, float v, int local) {
  if (local) *p = v;
  else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float xload(const float *p, int local) {
  return local ? *p : __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Placement check for the XCD-local exchange: a workgroup that does not run on
// XCD (blockIdx % 8) reports it (error bit 4) instead of combining silently.
__device__ __forceinline__ void check_xcd(int local, int *err, int lane) {
  if (local && lane == 0 && xcc_id() != int(blockIdx.x & 7)) atomicOr(err, 4);
}
// Completes this wave's exchange stores, then takes a ticket; true (uniform)
// for the last of `arrivals` arrivals, which then owns the combine and resets
// the counter for the next launch.
__device__ __forceinline__ bool last_arrival(unsigned *counter, unsigned arrivals, int lane) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  unsigned ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0);
  if (ticket != arrivals - 1) return false;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return true;
}
__device__ __forceinline__ void reset_counter(unsigned *counter, int lane) {
  if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// acc[m] = sum over s in slice order of part(s, m); PU independent loads per
// token in flight.
template <int MT, int PU, class AddrF>
__device__ __forceinline__ void sum_slices(float (&acc)[MT], AddrF part, int slices, int local) {
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
  for (int s0 = 0; s0 < slices; s0 += PU) {
    float v[PU][MT];
#pragma unroll
    for (int j = 0; j < PU; ++j)
      if (s0 + j < slices)
#pragma unroll
        for (int m = 0; m < MT; ++m) v[j][m] = xload(part(s0 + j, m), local);
#pragma unroll
    for (int j = 0; j < PU; ++j)
      if (s0 + j < slices)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] += v[j][m];
  }
}

// blockIdx -> (tile, rest): every workgroup of a tile goes to the same XCD
// (workgroups are dealt round-robin over the 8 XCDs), so the split-K partial
// sums of a tile stay in one L2.  `per` = workgroups per tile.
__device__ __forceinline__ bool map_tile(int b, int per, int tiles, int &tile, int &rest) {
  const int xcd = b & 7, k = b >> 3;
  const int q = k / per;
  tile = q * 8 + xcd;
  rest = k - q * per;
  return tile < tiles;
}

}  // namespace dev
}  // namespace qnn
