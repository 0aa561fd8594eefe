// qnn_int4.hip -- native INT4 (QuickNN group-32) kernels for gfx950.
//
// Format (src/core/QuickNN.Quantization.Int4.pas:10-94): per 32 weights an
// fp32 scale s then 16 bytes of offset-binary nibbles n (element j in byte j/2,
// low nibble for even j); value = fl32((n-8)*s).
//
// Device layout: see I4Layout in qnn_internal.h.  One wavefront owns a tile of
// 64 rows (one row per lane) and a K-slice of GS groups: every load is a
// 16-byte global_load_dwordx4 and consecutive lanes read consecutive 16-byte
// pieces, so each load instruction moves 1 KiB of packed weights.  The
// activation slice is staged in LDS with its per-group sums; the inner product
// folds the offset and scale per group:
//     sum_j (n_j - 8) s x_j = s * (sum_j n_j x_j - 8 * X_g),  X_g = sum_j x_j
// Slices of one tile are combined by the last wavefront to finish (an atomic
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

template <int MT, int GS>
__global__ __launch_bounds__(64) void k_int4_matvec(const I4Launch a, const int slices) {
  int tile, slice;
  if (!map_tile_slice(blockIdx.x, slices, a.tiles, tile, slice)) return;
  const int lane = threadIdx.x;
  const int g0 = slice * GS;
  const int ng = min(GS, a.g4 - g0);  // multiple of 4

  // 1) Issue every weight load of the slice first; HBM latency overlaps the
  //    activation staging below.  In I4_SWIGLU mode wave tile t covers output
  //    rows 32t..32t+31: lanes 0-31 read them from the gate matrix, lanes 32-63
  //    from the up matrix (rows (t&1)*32.. of stored tile t/2).
  int stile = tile, srow = lane;
  const void *nb = a.nib, *sb = a.scl;
  if (a.mode == I4_SWIGLU) {
    stile = tile >> 1;
    srow = (tile & 1) * 32 + (lane & 31);
    if (lane >= 32) { nb = a.nib2; sb = a.scl2; }
  }
  const uint4 *nib = static_cast<const uint4 *>(nb) + (size_t(stile) * a.g4 + g0) * 64 + srow;
  const float4 *scl = static_cast<const float4 *>(sb) + (size_t(stile) * (a.g4 >> 2) + (g0 >> 2)) * 64 + srow;
  uint4 w[GS];
  float4 s[GS / 4];
#pragma unroll
  for (int q = 0; q < GS / 4; ++q)
    if (4 * q < ng) s[q] = scl[q * 64];
#pragma unroll
  for (int g = 0; g < GS; ++g)
    if (g < ng) w[g] = nib[g * 64];

  // 2) Stage x[m][g0*32 .. g0*32+GS*32) and its per-group sums in LDS.
  __shared__ float xs[MT][GS * 32];
  __shared__ float xsum[MT][GS];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int it = 0; it < (GS + 7) / 8; ++it) {  // 256 floats per pass
      const int e = (it * 64 + lane) * 4;
      const int kk = g0 * 32 + e;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m < a.m && e < ng * 32) {
        const float *xr = a.x + size_t(m) * a.x_stride;
        if (kk + 3 < a.k) {
          v.x = xr[kk]; v.y = xr[kk + 1]; v.z = xr[kk + 2]; v.w = xr[kk + 3];
        } else {
          if (kk < a.k) v.x = xr[kk];
          if (kk + 1 < a.k) v.y = xr[kk + 1];
          if (kk + 2 < a.k) v.z = xr[kk + 2];
        }
      }
      if (e < GS * 32) *reinterpret_cast<float4 *>(&xs[m][e]) = v;
      float part = (v.x + v.y) + (v.z + v.w);
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      part += __shfl_xor(part, 4);
      if ((lane & 7) == 0 && e < GS * 32) xsum[m][e >> 5] = part;
    }
  }
  __syncthreads();

  // 3) Dequantise in registers and accumulate.
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int g = 0; g < GS; ++g) {
    if (g < ng) {
      const float sc = sel4(s[g >> 2], g & 3);
      float nv[32];  // nibble values of this group, element order
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t wd = sel4u(w[g], c);
        const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
          nv[c * 8 + 2 * bb] = float((lo >> (8 * bb)) & 0xFFu);
          nv[c * 8 + 2 * bb + 1] = float((hi >> (8 * bb)) & 0xFFu);
        }
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 *xv = reinterpret_cast<const float4 *>(&xs[m][g * 32]);
        float pc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float4 xa = xv[2 * c], xb = xv[2 * c + 1];
          float t = nv[c * 8] * xa.x;
          t = fmaf(nv[c * 8 + 1], xa.y, t);
          t = fmaf(nv[c * 8 + 2], xa.z, t);
          t = fmaf(nv[c * 8 + 3], xa.w, t);
          t = fmaf(nv[c * 8 + 4], xb.x, t);
          t = fmaf(nv[c * 8 + 5], xb.y, t);
          t = fmaf(nv[c * 8 + 6], xb.z, t);
          t = fmaf(nv[c * 8 + 7], xb.w, t);
          pc[c] = t;
        }
        const float pg = (pc[0] + pc[1]) + (pc[2] + pc[3]);
        acc[m] = fmaf(sc, pg - 8.0f * xsum[m][g], acc[m]);
      }
    }
  }

  // 4) Split-K combine: the last slice of a tile to finish sums all slices.
  //    Partials travel as device-scope atomic stores/loads, which are coherent
  //    across XCDs by themselves; the writer only has to wait for their
  //    completion before taking its ticket.  (A device-scope fence would write
  //    back and invalidate the whole L2 in every workgroup.)
  if (slices > 1) {
    float *part = a.partial + (size_t(tile) * slices + slice) * MT * 64;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      __hip_atomic_store(part + m * 64 + lane, acc[m], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // partial stores complete before the ticket
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    unsigned ticket = 0;
    if (lane == 0)
      ticket = __hip_atomic_fetch_add(&a.counters[tile * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = __shfl(ticket, 0);
    if (ticket != unsigned(slices - 1)) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    for (int s2 = 0; s2 < slices; ++s2) {
      const float *ps = a.partial + (size_t(tile) * slices + s2) * MT * 64;
#pragma unroll
      for (int m = 0; m < MT; ++m)
        acc[m] += __hip_atomic_load(ps + m * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) __hip_atomic_store(&a.counters[tile * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // 5) Epilogue.
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
void launch_mt(const I4Launch &a, int gs, int slices, int grid, hipStream_t st) {
  switch (gs) {
    case 4: hipLaunchKernelGGL((k_int4_matvec<MT, 4>), dim3(grid), dim3(64), 0, st, a, slices); break;
    case 8: hipLaunchKernelGGL((k_int4_matvec<MT, 8>), dim3(grid), dim3(64), 0, st, a, slices); break;
    case 16: hipLaunchKernelGGL((k_int4_matvec<MT, 16>), dim3(grid), dim3(64), 0, st, a, slices); break;
    default: hipLaunchKernelGGL((k_int4_matvec<MT, 32>), dim3(grid), dim3(64), 0, st, a, slices); break;
  }
}

int env_int(const char *name, int dflt) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

}  // namespace

void int4_plan(const I4Layout &l, int m, int *gs, int *slices) {
  const int tiles8 = (l.tiles + 7) / 8 * 8;
  const int target = env_int("QNN_I4_TARGET_WAVES", 2048);
  int forced = env_int("QNN_I4_GS", 0);
  int cap = m >= 8 ? 16 : 32;  // LDS and VGPR budget for many tokens
  int pick = 4;
  if (forced == 4 || forced == 8 || forced == 16 || forced == 32) {
    pick = std::min(forced, cap);
  } else {
    const int cands[] = {32, 16, 8};
    for (int c : cands) {
      if (c > cap) continue;
      if (size_t(tiles8) * ((l.g4 + c - 1) / c) >= size_t(target)) { pick = c; break; }
    }
  }
  *gs = pick;
  *slices = (l.g4 + pick - 1) / pick;
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
  else launch_mt<16>(a, std::min(gs, 16), slices, grid, st);
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
