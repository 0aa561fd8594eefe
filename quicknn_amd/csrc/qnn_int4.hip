// qnn_int4.hip -- native INT4 (QuickNN group-32) dense projection kernels for
// gfx950: matvec / multi-token matvec (Int4Linear, op 55/56), fused gate/up
// SwiGLU (op 68) and weighted accumulate (Int4LinearAccumulate, op 69), plus
// the repack and dequant kernels.  Format, layout and the fixed-point inner
// product: qnn_int4_dev.h.  Slices of one tile are combined by the last
// workgroup to finish (an atomic ticket per tile), in slice order, so results
// do not depend on timing.
#include "qnn_int4_dev.h"

namespace qnn {
namespace {
using dev::sel4u;

// Workgroup = 4 wavefronts on one 64-row tile and a K-slice of 4*GSW groups;
// the x slice is staged once per workgroup, the four partial sums meet in LDS.
// In I4_SWIGLU mode tile t covers output rows 32t..32t+31: lanes 0-31 read them
// from the gate matrix, lanes 32-63 from the up matrix (rows (t&1)*32.. of
// stored tile t/2).
template <int MT, int GSW>
__global__ __launch_bounds__(256) void k_int4_matvec(const I4Launch a, const int slices) {
  constexpr int GS = 4 * GSW;  // groups per workgroup slice
  int tile, slice;
  if (!dev::map_tile(blockIdx.x, slices, a.tiles, tile, slice)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g0 = slice * GS;
  const int ng = min(GS, a.g4 - g0);  // multiple of 4
  const int gw0 = wave * GSW;         // this wave's first group within the slice
  const int ngw = max(0, min(GSW, ng - gw0));

  // 1) Activation slice first (L2-resident, short latency), then this wave's
  //    weight stream.
  float4 xr[MT][dev::x_iters<GS>()];
  dev::load_x<MT, GS>(
      xr, [&](int m) -> const float * { return m < a.m ? a.x + size_t(m) * a.x_stride : nullptr; }, g0, ng, a.k,
      a.x_vec4 != 0, tid);
  int stile = tile, srow = lane;
  const void *nb = a.nib, *sb = a.scl;
  if (a.mode == I4_SWIGLU) {
    stile = tile >> 1;
    srow = (tile & 1) * 32 + (lane & 31);
    if (lane >= 32) { nb = a.nib2; sb = a.scl2; }
  }
  const int gq0 = g0 + gw0;  // first group of this wave (multiple of GSW)
  uint4 w[GSW];
  float sc[GSW];
  dev::load_w<GSW>(w, sc, static_cast<const uint4 *>(nb) + (size_t(stile) * a.g4 + gq0) * 64 + srow,
                   static_cast<const float *>(sb) + (size_t(stile) * (a.g4 >> 2) + (gq0 >> 2)) * 256 + srow * 4, gq0,
                   ngw);

  // 2) Fixed-point activation planes in LDS.
  __shared__ dev::XTile<MT, GS> xs;
  __shared__ float red[3][MT][64];
  dev::stage_x<MT, GS>(xs, xr, tid, lane);
  __syncthreads();

  // 3) Integer dot per group and token.
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
  dev::dot<MT, GS, GSW>(acc, w, sc, xs, gw0, ngw);

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
  //    slices in slice order.
  if (slices > 1) {
    float *part = a.partial + (size_t(tile) * slices + slice) * MT * 64;
    dev::check_xcd(a.xcd_local, a.err, lane);
#pragma unroll
    for (int m = 0; m < MT; ++m) dev::xstore(part + m * 64 + lane, acc[m], a.xcd_local);
    unsigned *ctr = &a.counters[tile * kCounterStride];
    if (!dev::last_arrival(ctr, unsigned(slices), lane)) return;
    const float *pt = a.partial + size_t(tile) * slices * MT * 64 + lane;
    constexpr int PU = MT >= 8 ? 2 : (MT >= 4 ? 4 : 16);  // independent partial loads in flight
    dev::sum_slices<MT, PU>(
        acc, [&](int s, int m) { return pt + (size_t(s) * MT + m) * 64; }, slices, a.xcd_local);
    dev::reset_counter(ctr, lane);
  }

  // 6) Epilogue.
  if (a.mode == I4_SWIGLU) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float u = __shfl_down(acc[m], 32);
      const int row = tile * 32 + lane;
      if (lane < 32 && row < a.n && m < a.m) a.y[size_t(m) * a.y_stride + row] = dev::silu(acc[m]) * u;
    }
  } else {
    const int row = tile * 64 + lane;
    if (row < a.n) {
      if (a.mode == I4_ACCUM) {
        a.y[row] = add_mul_nofma(a.y[row], acc[0], a.prob[0]);  // moe.comp:70
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
