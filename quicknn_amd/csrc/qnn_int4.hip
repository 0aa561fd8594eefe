// qnn_int4.hip -- native INT4 (QuickNN group-32) kernels for gfx950.
//
// Format (src/core/QuickNN.Quantization.Int4.pas:10-94): per 32 weights an
// fp32 scale s then 16 bytes of offset-binary nibbles n (element j in byte j/2,
// low nibble for even j); value = fl32((n-8)*s).
//
// Device layout: see I4Layout in qnn_internal.h.  One wavefront streams a tile
// of 64 rows (one row per lane): every load is a 16-byte global_load_dwordx4
// and consecutive lanes read consecutive 16-byte pieces, so each load
// instruction moves 1 KiB of packed weights.  The activation slice is staged
// in LDS as 16-bit fixed point per 32-group (two int8 planes); the inner
// product runs on the raw nibble bytes with v_dot4_i32_i8 and folds the
// offset and both scales once per group:
//     sum_j (n_j - 8) s x_j ~= s * s2 * (sum_j n_j (256 q1_j + q2_j) - 8 sum_j (256 q1_j + q2_j))
// (exact integer arithmetic inside a group; fp32 across groups; relative
// error of the activation representation <= 2^-16 of the group's max|x|).
// Slices of one tile are combined by the last workgroup to finish (an atomic
// ticket per tile), in slice order, so results do not depend on timing.
#include "qnn_internal.h"

namespace qnn {
namespace {

__device__ __forceinline__ float silu_dev(float g) {
  // Clamped SiLU of moe.comp:118 / QwenHybrid.CPU.pas:242-246.
  return g >= 20.0f ? g : (g <= -20.0f ? 0.0f : g / (1.0f + expf(-g)));
}

__device__ __forceinline__ float sel4(const float4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ uint32_t sel4u(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// blockIdx -> (tile, slice): all slices of a tile go to the same XCD
// (workgroups are dealt round-robin over the 8 XCDs), so the split-K partial
// sums of a tile stay in one L2.
__device__ __forceinline__ bool map_tile_slice(int b, int slices, int tiles, int &tile, int &slice) {
  const int xcd = b & 7, k = b >> 3;
  const int q = k / slices;
  tile = q * 8 + xcd;
  slice = k - q * slices;
  return tile < tiles;
}

// Workgroup = 4 wavefronts on one 64-row tile.  The workgroup owns a K-slice
// of 4*GSW groups; wave w streams groups [w*GSW, (w+1)*GSW) of it.  The x
// slice is staged once per workgroup; the four partial sums meet in LDS.
template <int MT, int GSW>
__global__ __launch_bounds__(256) void k_int4_matvec(const I4Launch a, const int slices) {
  constexpr int GS = 4 * GSW;  // groups per workgroup slice
  int tile, slice;
  if (!map_tile_slice(blockIdx.x, slices, a.tiles, tile, slice)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g0 = slice * GS;
  const int ng = min(GS, a.g4 - g0);  // multiple of 4
  const int gw0 = wave * GSW;         // this wave's first group within the slice
  const int ngw = max(0, min(GSW, ng - gw0));

  // 1) Activation slice first (L2-resident, short latency): 4 floats per
  //    thread per pass.  Then this wave's weight stream: scales, nibbles in
  //    group order.  Loads return in issue order, so group g is consumed as
  //    soon as it lands.  In I4_SWIGLU mode tile t covers output rows
  //    32t..32t+31: lanes 0-31 read them from the gate matrix, lanes 32-63
  //    from the up matrix (rows (t&1)*32.. of stored tile t/2).
  constexpr int XIT = (GS * 32 + 1023) / 1024;
  float4 xr_[MT][XIT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int e = (it * 256 + tid) * 4;
      const int kk = g0 * 32 + e;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m < a.m && e < ng * 32) {
        const float *xr = a.x + size_t(m) * a.x_stride;
        if (kk + 3 < a.k && a.x_vec4) {
          v = *reinterpret_cast<const float4 *>(xr + kk);
        } else if (kk + 3 < a.k) {
          v.x = xr[kk]; v.y = xr[kk + 1]; v.z = xr[kk + 2]; v.w = xr[kk + 3];
        } else {
          if (kk < a.k) v.x = xr[kk];
          if (kk + 1 < a.k) v.y = xr[kk + 1];
          if (kk + 2 < a.k) v.z = xr[kk + 2];
        }
      }
      xr_[m][it] = v;
    }
  }
  int stile = tile, srow = lane;
  const void *nb = a.nib, *sb = a.scl;
  if (a.mode == I4_SWIGLU) {
    stile = tile >> 1;
    srow = (tile & 1) * 32 + (lane & 31);
    if (lane >= 32) { nb = a.nib2; sb = a.scl2; }
  }
  const int gq0 = g0 + gw0;  // first group of this wave (multiple of GSW)
  const uint4 *nib = static_cast<const uint4 *>(nb) + (size_t(stile) * a.g4 + gq0) * 64 + srow;
  const float *sclf = static_cast<const float *>(sb) + (size_t(stile) * (a.g4 >> 2) + (gq0 >> 2)) * 256 + srow * 4;
  uint4 w[GSW];
  float sc[GSW];
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

  // 2) Quantise the x slice per 32-element group to 16-bit fixed point,
  //    x ~= s2 * (256*q1 + q2) with q1, q2 in [-127, 127]:
  //      s1 = amax/127, q1 = rint(x/s1), r = x - q1*s1, s2 = s1/256, q2 = rint(r/s2)
  //    (|x - s2(256 q1 + q2)| <= s2/2 = amax/65024).  The int8 planes are laid
  //    out to match the nibble bytes of a weight dword: dword c of a group
  //    holds elements 8c..8c+7, its low nibbles are the even elements and its
  //    high nibbles the odd ones, so word 2c packs x[8c+0,2,4,6] and word 2c+1
  //    x[8c+1,3,5,7].  Per group: 8 hi words, 8 lo words, s2 and -8*sum(q).
  __shared__ uint32_t xqh[MT][GS][8];
  __shared__ uint32_t xql[MT][GS][8];
  __shared__ float xs2[MT][GS];
  __shared__ int xoff[MT][GS];
  __shared__ float red[3][MT][64];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int e = (it * 256 + tid) * 4;  // first element of this thread, within the slice
      const float4 v = xr_[m][it];
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
        const int g = e >> 5, i0 = e & 31;  // i0 = 0 or 4 within dword c = i0/8... element 8c + (i0 & 7)
        const int c = i0 >> 3, half = (i0 >> 2) & 1;
        // bytes for even slots (elements +0, +2) and odd slots (+1, +3) of this half dword
        const uint32_t he = (uint32_t(h[0]) & 255u) | ((uint32_t(h[2]) & 255u) << 8);
        const uint32_t ho = (uint32_t(h[1]) & 255u) | ((uint32_t(h[3]) & 255u) << 8);
        const uint32_t le = (uint32_t(l[0]) & 255u) | ((uint32_t(l[2]) & 255u) << 8);
        const uint32_t lo = (uint32_t(l[1]) & 255u) | ((uint32_t(l[3]) & 255u) << 8);
        uint16_t *ph = reinterpret_cast<uint16_t *>(&xqh[m][g][0]);
        uint16_t *pl = reinterpret_cast<uint16_t *>(&xql[m][g][0]);
        ph[(2 * c) * 2 + half] = uint16_t(he);
        ph[(2 * c + 1) * 2 + half] = uint16_t(ho);
        pl[(2 * c) * 2 + half] = uint16_t(le);
        pl[(2 * c + 1) * 2 + half] = uint16_t(lo);
        if ((lane & 7) == 0) {
          xs2[m][g] = s1 * 0.00390625f;
          xoff[m][g] = -8 * sumq;
        }
      }
    }
  }
  __syncthreads();

  // 3) Dequantise-free integer dot: per group and token
  //    isum = 256 * dot(n, q1) + dot(n, q2) - 8 * sum(256 q1 + q2)  (exact, < 2^24)
  //    acc += float(isum) * (s * s2).
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
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
        const uint4 *qh = reinterpret_cast<const uint4 *>(&xqh[m][gl][0]);
        const uint4 *ql = reinterpret_cast<const uint4 *>(&xql[m][gl][0]);
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
        const int isum = ((ah0 + ah1) << 8) + (al0 + al1) + xoff[m][gl];
        acc[m] = fmaf(float(isum), sc[g] * xs2[m][gl], acc[m]);
      }
    }
  }

  // 4) Combine the four waves in LDS (fixed order: 0+1+2+3).
  if (wave > 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) red[wave - 1][m][lane] = acc[m];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = ((acc[m] + red[0][m][lane]) + red[1][m][lane]) + red[2][m][lane];

  // 5) Split-K across workgroups: the last slice of a tile to finish sums all
  //    slices in slice order.  Partials travel as device-scope atomic
  //    stores/loads, which are coherent across XCDs by themselves; the writer
  //    only waits for their completion before taking its ticket (a
  //    device-scope fence would write back and invalidate the whole L2).
  if (slices > 1) {
    float *part = a.partial + (size_t(tile) * slices + slice) * MT * 64;
    if (a.xcd_local) {
      // Every slice of this tile runs on XCD (blockIdx % 8); the partials meet
      // in that XCD's L2.  Verify the placement: a mismatch is reported, never
      // silently combined.
      if (lane == 0 && int(__builtin_amdgcn_s_getreg((3 << 11) | 20)) != int(blockIdx.x & 7)) atomicOr(a.err, 4);
#pragma unroll
      for (int m = 0; m < MT; ++m) part[m * 64 + lane] = acc[m];
    } else {
#pragma unroll
      for (int m = 0; m < MT; ++m)
        __hip_atomic_store(part + m * 64 + lane, acc[m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // partial stores complete before the ticket
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    unsigned ticket = 0;
    if (lane == 0)
      ticket = __hip_atomic_fetch_add(&a.counters[tile * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __shfl(ticket, 0);
    if (ticket != unsigned(slices - 1)) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const float *pt = a.partial + size_t(tile) * slices * MT * 64;
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    constexpr int PU = MT >= 8 ? 2 : (MT >= 4 ? 4 : 16);  // independent partial loads in flight
    for (int s0 = 0; s0 < slices; s0 += PU) {
      float v[PU][MT];
      if (a.xcd_local) {
#pragma unroll
        for (int j = 0; j < PU; ++j)
          if (s0 + j < slices)
#pragma unroll
            for (int m = 0; m < MT; ++m) v[j][m] = pt[(size_t(s0 + j) * MT + m) * 64 + lane];
      } else {
#pragma unroll
        for (int j = 0; j < PU; ++j)
          if (s0 + j < slices)
#pragma unroll
            for (int m = 0; m < MT; ++m)
              v[j][m] = __hip_atomic_load(pt + (size_t(s0 + j) * MT + m) * 64 + lane, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int j = 0; j < PU; ++j)
        if (s0 + j < slices)
#pragma unroll
          for (int m = 0; m < MT; ++m) acc[m] += v[j][m];
    }
    if (lane == 0) __hip_atomic_store(&a.counters[tile * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // 6) Epilogue.
  if (a.mode == I4_SWIGLU) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float u = __shfl_down(acc[m], 32);
      const int row = tile * 32 + lane;
      if (lane < 32 && row < a.n && m < a.m) a.y[size_t(m) * a.y_stride + row] = silu_dev(acc[m]) * u;
    }
  } else {
    const int row = tile * 64 + lane;
    if (row < a.n) {
      if (a.mode == I4_ACCUM) {
        a.y[row] = a.y[row] + acc[0] * a.prob[0];  // moe.comp:70
      } else {
#pragma unroll
        for (int m = 0; m < MT; ++m)
          if (m < a.m) a.y[size_t(m) * a.y_stride + row] = acc[m];
      }
    }
  }
}

// Raw packed rows -> tiled planes.  One thread per (tile, group, lane).
__global__ void k_int4_repack(const uint8_t *__restrict__ src, I4Layout l, uint4 *__restrict__ nib,
                              float *__restrict__ scl) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = size_t(l.tiles) * l.g4 * 64;
  if (idx >= total) return;
  const int r = int(idx & 63);
  const int g = int((idx >> 6) % l.g4);
  const int t = int(idx / (size_t(l.g4) * 64));
  const int srow = t * 64 + r;
  uint4 words = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
  float s = 0.0f;
  if (srow < l.rows && g < l.groups) {
    const uint8_t *blk = src + size_t(srow) * (size_t(l.groups) * 20) + size_t(g) * 20;
    const uint32_t *w32 = reinterpret_cast<const uint32_t *>(blk);  // 20-byte groups are 4-aligned
    s = __uint_as_float(w32[0]);
    words = make_uint4(w32[1], w32[2], w32[3], w32[4]);
  }
  nib[(size_t(t) * l.g4 + g) * 64 + r] = words;
  scl[((size_t(t) * (l.g4 >> 2) + (g >> 2)) * 64 + r) * 4 + (g & 3)] = s;
}

// Bit-exact dequantisation fl32((n-8)*s) of the resident tiled copy -> [rows][cols].
__global__ void k_int4_dequant(I4Layout l, const uint4 *__restrict__ nib, const float *__restrict__ scl,
                               float *__restrict__ out) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = size_t(l.rows) * l.cols;
  if (idx >= total) return;
  const int row = int(idx / l.cols), k = int(idx % l.cols);
  const int t = row / 64, r = row & 63;
  const int g = k >> 5, j = k & 31;
  const uint4 w = nib[(size_t(t) * l.g4 + g) * 64 + r];
  const uint32_t word = sel4u(w, j >> 3);
  const int n = int((word >> (4 * (j & 7))) & 15u);
  const float s = scl[((size_t(t) * (l.g4 >> 2) + (g >> 2)) * 64 + r) * 4 + (g & 3)];
  out[idx] = float(n - 8) * s;
}

template <int MT>
void launch_mt(const I4Launch &a, int gsw, int slices, int grid, hipStream_t st) {
  switch (gsw) {
    case 1: hipLaunchKernelGGL((k_int4_matvec<MT, 1>), dim3(grid), dim3(256), 0, st, a, slices); break;
    case 2: hipLaunchKernelGGL((k_int4_matvec<MT, 2>), dim3(grid), dim3(256), 0, st, a, slices); break;
    case 4: hipLaunchKernelGGL((k_int4_matvec<MT, 4>), dim3(grid), dim3(256), 0, st, a, slices); break;
    default: hipLaunchKernelGGL((k_int4_matvec<MT, 8>), dim3(grid), dim3(256), 0, st, a, slices); break;
  }
}

int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

}  // namespace

// Groups per wavefront (GSW); a workgroup slice is 4*GSW groups.  The default
// targets about 6k wavefronts per launch with at most ~40 slices per tile.
void int4_plan(const I4Layout &l, int m, int *gsw, int *slices) {
  const int tiles8 = (l.tiles + 7) / 8 * 8;
  const int target = env_int("QNN_I4_TARGET_WAVES", 3000);
  const int forced = env_int("QNN_I4_GSW", 0);
  const int cap = m >= 8 ? 4 : 8;  // LDS and VGPR budget for many tokens
  int pick = 1;
  if (forced == 1 || forced == 2 || forced == 4 || forced == 8) {
    pick = std::min(forced, cap);
  } else {
    const int cands[] = {4, 2};  // 8 groups per wave was never faster at M = 1
    for (int c : cands) {
      if (c > cap) continue;
      if (size_t(tiles8) * ((l.g4 + 4 * c - 1) / (4 * c)) * 4 >= size_t(target)) { pick = c; break; }
    }
  }
  *gsw = pick;
  *slices = (l.g4 + 4 * pick - 1) / (4 * pick);
}

size_t int4_partial_floats(const I4Layout &l, int m, int slices) {
  int mt = m <= 1 ? 1 : (m <= 2 ? 2 : (m <= 4 ? 4 : (m <= 8 ? 8 : 16)));
  return slices > 1 ? size_t(l.tiles) * slices * mt * 64 : 0;
}

void int4_matvec_launch(const I4Launch &a, int gs, int slices, hipStream_t st) {
  const int tiles8 = (a.tiles + 7) / 8 * 8;
  const int grid = tiles8 * slices;
  if (a.m <= 1) launch_mt<1>(a, gs, slices, grid, st);
  else if (a.m <= 2) launch_mt<2>(a, gs, slices, grid, st);
  else if (a.m <= 4) launch_mt<4>(a, gs, slices, grid, st);
  else if (a.m <= 8) launch_mt<8>(a, gs, slices, grid, st);
  else launch_mt<16>(a, std::min(gs, 4), slices, grid, st);
  hip_check(hipGetLastError(), "int4 matvec launch");
}

I4Layout int4_layout(int rows, int cols) {
  I4Layout l;
  l.rows = rows;
  l.cols = cols;
  l.groups = (cols + 31) / 32;
  l.g4 = (l.groups + 3) / 4 * 4;
  l.tiles = (rows + 63) / 64;
  return l;
}

void int4_repack_launch(const uint8_t *src, const I4Layout &l, void *dst, hipStream_t st) {
  const size_t total = size_t(l.tiles) * l.g4 * 64;
  uint4 *nib = static_cast<uint4 *>(dst);
  float *scl = reinterpret_cast<float *>(static_cast<uint8_t *>(dst) + l.nib_bytes());
  hipLaunchKernelGGL(k_int4_repack, dim3((total + 255) / 256), dim3(256), 0, st, src, l, nib, scl);
  hip_check(hipGetLastError(), "int4 repack launch");
}

void int4_dequant_launch(const I4Layout &l, const void *w, float *out, hipStream_t st) {
  const size_t total = size_t(l.rows) * l.cols;
  const uint4 *nib = static_cast<const uint4 *>(w);
  const float *scl = reinterpret_cast<const float *>(static_cast<const uint8_t *>(w) + l.nib_bytes());
  hipLaunchKernelGGL(k_int4_dequant, dim3((total + 255) / 256), dim3(256), 0, st, l, nib, scl, out);
  hip_check(hipGetLastError(), "int4 dequant launch");
}

}  // namespace qnn
