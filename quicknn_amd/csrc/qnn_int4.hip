// qnn_int4.hip -- native INT4 (QuickNN group-32) dense projection kernels for
// gfx950: matvec / multi-token matvec (Int4Linear, op 55/56), fused gate/up
// SwiGLU (op 68) and weighted accumulate (Int4LinearAccumulate, op 69), plus
// the repack and dequant kernels.  Format, layout and the fixed-point inner
// product: qnn_int4_dev.h.
//
// A workgroup is 4 waves: T consecutive tiles (64-lane blocks; in SwiGLU mode
// half a block of gate rows in lanes 0-31 and the same up rows in lanes 32-63)
// times P = 4/T parts of one K-slice, each part `steps_per_slice` steps long.
// The workgroup's activation slice is staged once in LDS for all four waves.
// Each lane accumulates its groups, the L lanes of a row are reduced across
// the wave, the P parts of a tile are summed in LDS by part 0, and when the
// K-range is split over several workgroups the last slice of a tile to finish
// (an atomic ticket per tile) sums the slices in slice order, so results do not
// depend on timing.  The planner (int4_plan) picks 4 steps per wave for one
// token; for several, the largest power-of-two that splits the steps evenly
// and still gives enough waves to fill the chip.  With 4-16 tokens over
// one-lane rows at 4 steps per wave the group dots run on the int8 matrix
// cores (dot_mf), bit-identical to the v_dot4 path.
#include "qnn_int4_dev.h"

namespace qnn {
namespace {
using dev::sel4u;

// One tile per workgroup (four parts) and 4-16 tokens: the same sums as
// below, spread over the four waves.  Every part goes to LDS; wave w then
// owns tokens w*MT/4 .. (w+1)*MT/4-1: it sums their four parts (order
// 0+1+2+3), stores their partials, and, when the workgroup's ticket is the
// last, sums their slices (slice order) and writes their outputs.  The
// combine's loads are spread over four waves instead of one, so they go out
// in one or two batches instead of up to five.
template <int MT>
__device__ __forceinline__ void finish_tile_wide(const I4Launch &a, float (&acc)[MT], float (*red)[MT][64], int wave,
                                                 int lane, int tile, int slice, int slices, int b, bool active) {
  constexpr int TW = MT / 4;                                  // tokens per wave
  constexpr int PS = TW == 1 ? 32 : (TW == 2 ? 20 : 8);       // slices per batch of loads, one matrix
  constexpr int PG = TW == 1 ? 16 : (TW == 2 ? 8 : 4);        // slices per batch, gate and up
  __shared__ int last_wg;
  const I4Layout &l = a.l;
  const bool swiglu = a.mode == I4_SWIGLU;
#pragma unroll
  for (int m = 0; m < MT; ++m) red[wave][m][lane] = acc[m];
  __syncthreads();
  if (!active) return;  // uniform: one tile per workgroup
  const int m0 = wave * TW;
  float v[TW], vu[TW];
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    v[i] = red[0][m0 + i][lane];
    v[i] += red[1][m0 + i][lane];
    v[i] += red[2][m0 + i][lane];
    v[i] += red[3][m0 + i][lane];
  }
  if (slices > 1 || swiglu) {
    float *part_p = a.partial + (size_t(tile) * slices + slice) * MT * 64 + lane;
#pragma unroll
    for (int i = 0; i < TW; ++i) dev::xstore(part_p + (m0 + i) * 64, v[i]);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partials are at the coherence point
    __syncthreads();
    unsigned *ctr = &a.counters[size_t(swiglu ? tile >> 1 : tile) * kCounterStride];
    if (wave == 0) {
      const bool last = dev::last_arrival(ctr, unsigned(swiglu ? 2 * slices : slices), lane);
      if (lane == 0) last_wg = last ? 1 : 0;
    }
    __syncthreads();
    if (!last_wg) return;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int t0 = swiglu ? tile & ~1 : tile;
    const float *pt = a.partial + size_t(t0) * slices * MT * 64 + lane;
    if (swiglu) {  // gate and up partials of this wave's tokens in one batch
      const float *pu = pt + size_t(slices) * MT * 64;
      float gu[2 * TW];
      dev::sum_slices<2 * TW, PG>(
          gu, [&](int s, int i) { return (i < TW ? pt : pu) + (size_t(s) * MT + m0 + (i < TW ? i : i - TW)) * 64; },
          slices);
#pragma unroll
      for (int i = 0; i < TW; ++i) {
        v[i] = gu[i];
        vu[i] = gu[TW + i];
      }
    } else {
      dev::sum_slices<TW, PS>(
          v, [&](int s, int i) { return pt + (size_t(s) * MT + m0 + i) * 64; }, slices);
    }
    if (wave == 0) dev::reset_counter(ctr, lane);
  }
  // Epilogue: the first lane of each row writes this wave's tokens of it.
  const int row = b * l.rpb + lane / l.lanes;
  if ((lane & (l.lanes - 1)) != 0 || row >= a.n) return;
#pragma unroll
  for (int i = 0; i < TW; ++i) {
    const int m = m0 + i;
    if (m >= a.m) continue;
    if (swiglu) {
      if (a.g_out) {
        a.g_out[size_t(m) * a.y_stride + row] = v[i];
        a.u_out[size_t(m) * a.y_stride + row] = vu[i];
      }
      a.y[size_t(m) * a.y_stride + row] = dev::silu(v[i]) * vu[i];
    } else {
      a.y[size_t(m) * a.y_stride + row] = v[i];
    }
  }
}

// The P parts of a tile meet in LDS (part 0 sums them in order 0+1+2+3),
// then the split-K exchange and the epilogue.
template <int MT, int P>
__device__ __forceinline__ void finish_tile(const I4Launch &a, float (&acc)[MT], float (*red)[MT][64], int wave,
                                            int part, int lane, int tile, int slice, int slices, int b, bool active) {
  const I4Layout &l = a.l;
  const bool swiglu = a.mode == I4_SWIGLU;
  const int L = l.lanes, j = lane & (L - 1), wl = lane;
  if constexpr (P == 4 && MT >= 4) {
    if (a.mode != I4_ACCUM) {
      finish_tile_wide<MT>(a, acc, red, wave, lane, tile, slice, slices, b, active);
      return;
    }
  }
  if (P > 1) {
    if (part > 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m) red[wave][m][lane] = acc[m];
    }
    __syncthreads();
    if (part > 0) return;
    if constexpr (P <= 4) {
#pragma unroll
      for (int q = 1; q < P; ++q)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] += red[wave + q][m][lane];
    } else {
      // An 8- or 16-wave workgroup over the whole K-range: its parts are
      // summed as P / 4 four-wave slices and their split-K combine would sum
      // them (four parts in order, then the slices in order from zero), so
      // the result is the same bit for bit.
      float tot[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) tot[m] = 0.0f;
#pragma unroll
      for (int g = 0; g < P / 4; ++g)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float q = g == 0 ? acc[m] : red[wave + 4 * g][m][lane];
#pragma unroll
          for (int r = 1; r < 4; ++r) q += red[wave + 4 * g + r][m][lane];
          tot[m] += q;
        }
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[m] = tot[m];
    }
  }
  if (!active) return;

  // 4) Split-K across workgroups: the last slice of a tile to finish sums all
  //    slices in slice order.  I4_SWIGLU always meets here: the last of the
  //    2 x slices arrivals of a block sums the gate slices and the up slices.
  constexpr int PU = MT >= 16 ? 2 : (MT >= 8 ? 4 : (MT >= 4 ? 8 : 16));  // independent partial loads in flight
  float accu[MT];
  if (slices > 1 || swiglu) {
    float *part_p = a.partial + (size_t(tile) * slices + slice) * MT * 64 + lane;
#pragma unroll
    for (int m = 0; m < MT; ++m) dev::xstore(part_p + m * 64, acc[m]);
    unsigned *ctr = &a.counters[size_t(swiglu ? tile >> 1 : tile) * kCounterStride];
    if (!dev::last_arrival(ctr, unsigned(swiglu ? 2 * slices : slices), lane)) return;
    const int t0 = swiglu ? tile & ~1 : tile;
    const float *pt = a.partial + size_t(t0) * slices * MT * 64 + lane;
    if (swiglu) {  // gate and up partials in one batch of loads
      const float *pu = pt + size_t(slices) * MT * 64;
      float gu[2 * MT];
      dev::sum_slices<2 * MT, (PU > 1 ? PU / 2 : 1)>(  // as many loads in flight as one matrix at PU
          gu, [&](int s, int m) { return (m < MT ? pt : pu) + (size_t(s) * MT + (m < MT ? m : m - MT)) * 64; },
          slices);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        acc[m] = gu[m];
        accu[m] = gu[MT + m];
      }
    } else {
      dev::sum_slices<MT, PU>(
          acc, [&](int s, int m) { return pt + (size_t(s) * MT + m) * 64; }, slices);
    }
    dev::reset_counter(ctr, lane);
  }

  // 5) Epilogue: the first lane of each row writes it.
  if (swiglu) {
    const int row = b * l.rpb + wl / L;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (j == 0 && row < a.n && m < a.m) {
        if (a.g_out) {
          a.g_out[size_t(m) * a.y_stride + row] = acc[m];
          a.u_out[size_t(m) * a.y_stride + row] = accu[m];
        }
        a.y[size_t(m) * a.y_stride + row] = dev::silu(acc[m]) * accu[m];
      }
  } else {
    const int row = b * l.rpb + lane / L;
    if (j == 0 && row < a.n) {
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

// MF: the inner product on the int8 matrix cores (dot_mf; L = 1, MT >= 4,
// GSW a multiple of 4), bit-identical to the v_dot4 path.
// W = 4 waves per workgroup, or (one token, one tile, I4_STORE) 8 or 16: one
// workgroup over a K-range that two or four four-wave slices would split, so
// its parts meet in LDS instead of in a cross-workgroup exchange.
template <int MT, int GSW, int T, bool MF, int W = 4>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(MF ? (MT <= 8 ? 6 : 5) : 1)))
void k_int4_matvec(const I4Launch a, const int slices) {
  static_assert(W == 4 || (MT == 1 && T == 1 && !MF && (W == 8 || W == 16)), "wide workgroups: one token, one tile");
  extern __shared__ uint4 dyn_lds[];
  __shared__ float red[W][MT][64];
  constexpr int P = W / T;  // waves per tile: parts of the workgroup's K-slice
  const int wave = dev::wave_id(), tid = threadIdx.x, lane = tid & 63;
  const bool swiglu = a.mode == I4_SWIGLU;
  // I4_SWIGLU with one tile per workgroup: units are padded to groups of 16 so
  // that the gate tile (unit u) and the up tile (unit u + 8) of a block land on
  // one XCD; with T >= 2 they share the workgroup.
  const int units = swiglu && T == 1 ? (a.tiles + 15) / 16 * 16 : (a.tiles + T - 1) / T;
  int unit, slice;
  if (!dev::map_tile(blockIdx.x, slices, units, unit, slice)) return;
  const I4Layout &l = a.l;
  const int L = l.lanes, j = lane & (L - 1);
  const int sps = a.steps_per_slice;  // steps per wave
  const int part = wave % P;
  const int ws0 = slice * P * sps;                     // first step of the workgroup's slice
  const int s0 = ws0 + part * sps;                     // first step of this wave
  const int ns = max(0, min(sps, l.steps - s0));
  const int sgroups = min(P * sps * L, l.groups - ws0 * L);  // groups of x in the slice

  // 1) Activation slice first (L2-resident, short latency), then this wave's
  //    weight stream.  All loads are unconditional (buffer loads past the end
  //    return 0); a wave past the last tile reads tile 0 and stops after the
  //    barrier.
  // The slice is P*sps*L <= 16*GSW groups (the planner keeps P*L <= 16).
  // MF: slices of at most 4 x 4 x 32 = 512 elements, staged four tokens per pass.
  float4 xr[MF ? 1 : MT][MF ? 1 : dev::x_iters<GSW>()];
  float4 xr4[MF ? MT / 4 : 1][2];
  const dev::Rsrc xsrc = dev::rsrc(a.x, size_t(a.m) * a.x_stride * 4);
  auto xrow = [&](int m) { return uint32_t(m) * uint32_t(a.x_stride) * 4u; };
  // (Wide workgroups: the first four waves load and stage the slice, which
  // the planner keeps within their x_iters passes.)
  const bool xstager = W == 4 || tid < 256;
  if constexpr (MF)
    dev::load_x_quads<MT>(xr4, xsrc, xrow, a.m, ws0 * L * 32, wave, lane);
  else if (xstager)
    dev::load_x<MT, GSW>(xr, xsrc, xrow, a.m, ws0 * L * 32, sgroups * 32, tid);
  int tile = unit * T + wave / P;
  if (swiglu && T == 1) tile = 2 * ((unit >> 4) * 8 + (unit & 7)) + ((unit >> 3) & 1);
  const bool active = tile < a.tiles;
  const int t = active ? tile : 0;
  // I4_SWIGLU: tile 2b is the gate matrix's block b, tile 2b + 1 the up
  // matrix's; the choice is uniform per wave, so the buffer resources stay
  // scalar.
  int b = t;
  const int wl = lane;
  const void *nb = a.nib, *sb = a.scl;
  if (swiglu) {
    b = t >> 1;
    if (t & 1) { nb = a.nib2; sb = a.scl2; }
  }
  uint4 w[MF ? 1 : GSW];
  float sc[MF ? 1 : GSW];
  dev::MfWeights<MF ? GSW : 4> mw;
  const dev::XPlanes xs = dev::xplanes_at(dyn_lds, MT, P * sps * L);
  // 2) Fixed-point activation planes in LDS.  On the matrix-core path (4-16
  //    tokens) the slice is staged before the weight loads are issued: a
  //    wave cannot pass its weight loads until the memory pipeline accepts
  //    them, which under the whole grid's stream took microseconds (batch-8
  //    gate/up 18.8 -> 17.5 us, down 13.1 -> 12.2 us).  With one token the
  //    staging is short and issuing the weights first is faster (6144 x 2048
  //    5.9 against 6.3 us).
  if constexpr (MF) {
    dev::stage_x_quads<MT>(xs, xr4, a.m, ws0 * L * 32, sgroups * 32, a.k, wave, lane);
    dev::load_w_mf<GSW>(mw, dev::block_nib_rsrc(nb, l, b), dev::block_scl_rsrc(sb, l, b), l, b, s0, lane);
  } else {
    dev::load_w<GSW>(w, sc, dev::block_nib_rsrc(nb, l, b), dev::block_scl_rsrc(sb, l, b), l, b, s0, wl);
    if (xstager) dev::stage_x<MT, GSW>(xs, xr, a.m, ws0 * L * 32, sgroups * 32, a.k, tid, lane);
  }
  __syncthreads();

  // 3) Integer dot per group and token, the L lanes of each row, then the P
  //    parts of each tile (fixed order 0+1+2+3).
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
  if (active && ns > 0) {
    dev::XPlanes xp = xs;
    const int g0 = part * sps * L;
    xp.q = xs.q + size_t(g0) * dev::kXWords;
    xp.s2 = xs.s2 + g0;
    xp.off = xs.off + g0;
    if constexpr (MF) {
      float accm[4][dev::mf_per_lane<MT>()];
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
#pragma unroll
        for (int r = 0; r < dev::mf_per_lane<MT>(); ++r) accm[rq][r] = 0.0f;
      dev::dot_mf<MT, GSW>(accm, mw, xp, ns, lane);
      dev::mf_to_rows<MT>(acc, accm, &red[wave][0][0], lane);
    } else {
      dev::dot<MT, GSW>(acc, w, sc, xp, L, j, ns);
      dev::reduce_lanes<MT>(acc, L);
    }
  }
  finish_tile<MT, P>(a, acc, red, wave, part, lane, tile, slice, slices, b, active);
}

// Raw packed rows -> device layout.  One thread per (block, step, lane).
__global__ void k_int4_repack(const uint8_t *__restrict__ src, I4Layout l, uint4 *__restrict__ nib,
                              float *__restrict__ scl) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = size_t(l.blocks) * l.steps * 64;
  if (idx >= total) return;
  const int lane = int(idx & 63);
  const int s = int((idx >> 6) % l.steps);
  const int b = int(idx / (size_t(l.steps) * 64));
  const int row = b * l.rpb + lane / l.lanes, g = s * l.lanes + (lane & (l.lanes - 1));
  uint4 words = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
  float sv = 0.0f;
  if (row < l.rows && g < l.groups) {
    const uint8_t *blk = src + size_t(row) * (size_t(l.groups) * 20) + size_t(g) * 20;
    const uint32_t *w32 = reinterpret_cast<const uint32_t *>(blk);  // 20-byte groups are 4-aligned
    sv = __uint_as_float(w32[0]);
    words = make_uint4(w32[1], w32[2], w32[3], w32[4]);
  }
  nib[idx] = words;
  scl[l.scale_at(b, s, lane)] = sv;
  if (s == l.steps - 1)  // the last piece's slots past the last step hold 0
    for (int p = s + 1; p < l.quads() * 4; ++p) scl[l.scale_at(b, p, lane)] = 0.0f;
}

// Bit-exact dequantisation fl32((n-8)*s) of the resident copy -> [rows][cols].
__global__ void k_int4_dequant(I4Layout l, const uint4 *__restrict__ nib, const float *__restrict__ scl,
                               float *__restrict__ out) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = size_t(l.rows) * l.cols;
  if (idx >= total) return;
  const int row = int(idx / l.cols), k = int(idx % l.cols);
  const int b = row / l.rpb, r = row % l.rpb;
  const int g = k >> 5, e = k & 31;
  const int s = g / l.lanes, lane = r * l.lanes + (g & (l.lanes - 1));
  const size_t at = (size_t(b) * l.steps + s) * 64 + lane;
  const uint32_t word = sel4u(nib[at], e >> 3);
  const int n = int((word >> (4 * (e & 7))) & 15u);
  out[idx] = float(n - 8) * scl[l.scale_at(b, s, lane)];
}

template <int MT, int GSW, bool MF>
void launch_tpw(const I4Launch &a, const I4Plan &p, hipStream_t st) {
  if constexpr (MT == 1 && !MF) {
    if (p.wg_waves == 16) {
      hipLaunchKernelGGL((k_int4_matvec<1, GSW, 1, false, 16>), dim3(p.grid), dim3(1024), p.lds, st, a, p.slices);
      return;
    }
    if (p.wg_waves == 8) {
      hipLaunchKernelGGL((k_int4_matvec<1, GSW, 1, false, 8>), dim3(p.grid), dim3(512), p.lds, st, a, p.slices);
      return;
    }
  }
  if (p.wg_waves != 4) fail(QNN_E_INVALID_OP, "int4 plan: wide workgroups take one token");
  switch (p.tiles_per_wg) {
    case 1: hipLaunchKernelGGL((k_int4_matvec<MT, GSW, 1, MF>), dim3(p.grid), dim3(256), p.lds, st, a, p.slices); break;
    case 2: hipLaunchKernelGGL((k_int4_matvec<MT, GSW, 2, MF>), dim3(p.grid), dim3(256), p.lds, st, a, p.slices); break;
    default: hipLaunchKernelGGL((k_int4_matvec<MT, GSW, 4, MF>), dim3(p.grid), dim3(256), p.lds, st, a, p.slices); break;
  }
}
// Several tokens over one-lane rows with 4 steps per wave: the matrix-core
// inner product (QNN_I4_MFMA=0 keeps v_dot4).
bool mfma_enabled() { return tuning().i4_mfma != 0; }

template <int MT, int GSW>
void launch_one(const I4Launch &a, const I4Plan &p, hipStream_t st) {
  if constexpr (MT >= 4 && GSW == 4) {
    if (a.l.lanes == 1 && mfma_enabled()) {
      launch_tpw<MT, GSW, true>(a, p, st);
      return;
    }
  }
  if constexpr (MT == 16 && GSW == 4)  // planned only for the matrix-core path
    fail(QNN_E_INVALID_OP, "int4 plan: 16 tokens at 4 steps per wave without the matrix cores");
  else
    launch_tpw<MT, GSW, false>(a, p, st);
}

// Steps-per-wave templates by token count (register budget).
constexpr int kGsw1[] = {1, 2, 4, 8};
constexpr int kGswN[] = {1, 2, 4};
constexpr int kGswBig[] = {1, 2, 4};

template <int MT>
void launch_mt(const I4Launch &a, const I4Plan &p, hipStream_t st) {
  switch (p.gsw) {
    case 1: launch_one<MT, 1>(a, p, st); return;
    case 2: launch_one<MT, 2>(a, p, st); return;
    default: break;
  }
  if (p.gsw == 4) {  // 16 tokens: matrix cores only
    launch_one<MT, 4>(a, p, st);
    return;
  }
  if constexpr (MT == 1) {
    if (p.gsw == 8) {
      launch_one<1, 8>(a, p, st);
      return;
    }
  }
  fail(QNN_E_INVALID_OP, "int4 plan: steps per wave");
}

int pick_template(int sps, const int *set, int n) {
  for (int i = 0; i < n; ++i)
    if (set[i] >= sps) return set[i];
  return set[n - 1];
}

}  // namespace

I4Layout int4_layout(int rows, int cols, bool one_lane) {
  I4Layout l;
  l.rows = rows;
  l.cols = cols;
  l.groups = (cols + 31) / 32;
  // Lanes per row: 1 (a wave streams 64 rows, one per lane, and all lanes
  // share each activation group), measured fastest at the decode shapes.
  // QNN_I4_LANES selects 2..16 lanes per row instead.
  l.lanes = 1;
  const int forced = tuning().i4_lanes;
  if (!one_lane && (forced == 1 || forced == 2 || forced == 4 || forced == 8 || forced == 16)) l.lanes = forced;
  l.rpb = 64 / l.lanes;
  l.steps = (l.groups + l.lanes - 1) / l.lanes;
  l.blocks = (rows + l.rpb - 1) / l.rpb;
  return l;
}

I4Plan int4_plan(const I4Layout &l, int m, int mode, bool wide) {
  I4Plan p;
  p.mt = m <= 1 ? 1 : (m <= 2 ? 2 : (m <= 4 ? 4 : (m <= 8 ? 8 : 16)));
  const int tiles = mode == I4_SWIGLU ? 2 * l.blocks : l.blocks;
  // Tiles per workgroup (the other 4/T waves of a tile split its K-slice and
  // meet in LDS before any cross-workgroup exchange).
  const int ft = tuning().i4_tpw;
  p.tiles_per_wg = ft == 2 || ft == 4 ? ft : 1;
  while (p.tiles_per_wg < 4 && (4 / p.tiles_per_wg) * l.lanes > 16) p.tiles_per_wg *= 2;  // slice fits x_iters
  const int P = 4 / p.tiles_per_wg;
  // Steps per wave: bounded by the template set (registers) and by the LDS of
  // the workgroup's activation slice (at most 48 KiB).  One token: 4 steps
  // per wave whatever the wave count.  Fewer steps give more waves but more
  // split-K arrivals per tile, and at batch 1 the exchange costs more than
  // the waves gain: 4 against the 1-2 a 3000-wave target picks was 5-16%
  // faster at every measured decode shape (6144x2048 6.58 -> 6.18 us,
  // 2560x2560 6.42 -> 5.38, 1024x2560 5.83 -> 4.97), and 8 was slower.
  const int set_max = p.mt <= 8 || (l.lanes == 1 && mfma_enabled()) ? 4 : 2;  // 16 tokens: 4 on the matrix cores
  const int lds_max = int((48 << 10) / (size_t(p.mt) * P * l.lanes * (dev::kXWords * 4 + 8)));
  const int cap = std::max(1, std::min(set_max, lds_max));
  // Steps per wave: the largest that splits the K-range into equal workgroup
  // slices (an uneven last slice was measured up to 40% slower) while giving
  // at least `target` waves; failing that, the largest that gives the waves.
  const int target = tuning().i4_target_waves > 0 ? tuning().i4_target_waves : (p.mt == 1 ? 1 : 3000);
  const int units = (tiles + p.tiles_per_wg - 1) / p.tiles_per_wg;
  auto waves = [&](int sps) { return size_t(units) * 4 * ((l.steps + P * sps - 1) / (P * sps)); };
  const int *set0 = p.mt == 1 ? kGsw1 : (p.mt <= 4 ? kGswN : kGswBig);
  const int nset0 = p.mt == 1 ? int(sizeof kGsw1 / sizeof(int)) : 3;
  int sps = 0;
  for (int i = nset0 - 1; i >= 0 && !sps; --i)
    if (set0[i] <= cap && l.steps % (P * set0[i]) == 0 && waves(set0[i]) >= size_t(target)) sps = set0[i];
  for (int i = nset0 - 1; i >= 0 && !sps; --i)
    if (set0[i] <= cap && waves(set0[i]) >= size_t(target)) sps = set0[i];
  if (!sps) sps = 1;
  const int forced = tuning().i4_sps;
  if (forced > 0) {  // a power of two: scale pieces hold 4 aligned steps
    sps = 1;
    while (sps * 2 <= std::min(forced, cap)) sps *= 2;
  }
  const int *set = p.mt == 1 ? kGsw1 : (p.mt <= 4 ? kGswN : kGswBig);
  const int nset = p.mt == 1 ? int(sizeof kGsw1 / sizeof(int)) : 3;
  sps = std::min(sps, pick_template(sps, set, nset));
  p.gsw = pick_template(sps, set, nset);
  p.steps_per_slice = sps;
  p.slices = (l.steps + P * sps - 1) / (P * sps);
  p.lds = dev::xplanes_bytes(p.mt, P * sps * l.lanes);
  const int grid_units = mode == I4_SWIGLU && p.tiles_per_wg == 1 ? (tiles + 15) / 16 * 16 : (units + 7) / 8 * 8;
  p.grid = grid_units * p.slices;
  // One token over one-lane rows whose K-range splits evenly into 2 or 4
  // four-wave slices: one 8- or 16-wave workgroup per tile instead, with no
  // cross-workgroup exchange (QNN_I4_WIDE=0 keeps the slices).  Only where
  // the caller launches k_int4_matvec (`wide`): the fused MLP builds its down
  // items from the four-wave slices.
  if (wide && mode == I4_STORE && p.mt == 1 && p.tiles_per_wg == 1 && l.lanes == 1 && (p.slices == 2 || p.slices == 4) &&
      l.steps == P * sps * p.slices && tuning().i4_wide != 0) {
    p.wg_waves = 4 * p.slices;
    p.slices = 1;
    p.lds = dev::xplanes_bytes(p.mt, p.wg_waves * sps * l.lanes);
    p.grid = grid_units;
  }
  p.partial_floats = p.slices > 1 || mode == I4_SWIGLU ? size_t(tiles) * p.slices * p.mt * 64 : 0;
  p.counters = size_t(tiles) * kCounterStride;
  return p;
}

void int4_matvec_launch(const I4Launch &a0, const I4Plan &p, hipStream_t st) {
  I4Launch a = a0;
  a.steps_per_slice = p.steps_per_slice;
  if (p.mt == 1) launch_mt<1>(a, p, st);
  else if (p.mt == 2) launch_mt<2>(a, p, st);
  else if (p.mt == 4) launch_mt<4>(a, p, st);
  else if (p.mt == 8) launch_mt<8>(a, p, st);
  else launch_mt<16>(a, p, st);
  hip_check(hipGetLastError(), "int4 matvec launch");
}

void int4_repack_launch(const uint8_t *src, const I4Layout &l, void *dst, hipStream_t st) {
  const size_t total = size_t(l.blocks) * l.steps * 64;
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
