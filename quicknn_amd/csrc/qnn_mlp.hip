// qnn_mlp.hip -- one native-INT4 decode MLP (fused gate/up SwiGLU, then down)
// in a single launch.
//
// The engine issues TrySwiGLUVector (op 68) and then Int4Linear (op 55) on
// its output for every layer (src/models/QuickNN.Models.QwenHybrid.CPU.pas:
// 238-248 is the same composition on the CPU).  As two launches, the down
// projection cannot start streaming its weights before the gate/up launch has
// drained, and each launch pays its own ramp-up and split-K tail while HBM
// idles.  Here every workgroup issues its down-projection weight loads as
// soon as its gate/up item is done, so the layer's weights stream as one with
// every gate/up weight requested first (h completes sooner), and each down
// item starts as soon as the part of h it reads exists.
//
// Work items are exactly those of the two per-op launches (qnn_int4.hip):
// gate/up items (tile, slice) of the I4_SWIGLU plan and down items of the
// I4_STORE plan, with the same per-wave steps, the same in-workgroup order and
// the same slice order, so h and y are bit-identical to the per-op path.
// Workgroup w runs gate/up item w, then (for w below the down grid) down item
// w, each placed with the per-op kernels' tile map (qnn_exchange.h).
//
// Dataflow instead of a barrier: the workgroup that completes a block of h
// (64 rows) writes it with device-coherent stores and then sets that block's
// flag to the launch's epoch (flags 256 B apart, never reset: a stale flag
// holds an older epoch).  A down item reads 8 blocks of h (its K-slice), so it
// waits for those 8 flags only; nothing waits on a word that every workgroup
// touches (atomics and polls on one word serialise at its memory channel).
// Gate/up items never wait, so with every workgroup resident (the grid never
// exceeds the co-resident count) all waits end; they are bounded anyway: on
// timeout the error word gets bit 2 and the kernel finishes.
#include "qnn_int4_dev.h"

namespace qnn {
namespace {

// Phase timestamps, built only into libqnn_hip_trace.so (-DQNN_PHASE_TRACE):
// thread 0 of workgroup wg stores the device's real-time counter (100 MHz)
// when it reaches phase k of the fused kernels; qnn_phase_trace reads them.
// Nothing else changes: the same work runs in the same order.
#ifdef QNN_PHASE_TRACE
constexpr int kPhaseWGs = 2048, kPhases = 16;
__device__ unsigned long long g_phase[kPhaseWGs * kPhases];
#define QNN_PHASE(k)                                                                                 \
  do {                                                                                               \
    if (threadIdx.x == 0 && blockIdx.x < kPhaseWGs)                                                  \
      g_phase[blockIdx.x * kPhases + (k)] = __builtin_amdgcn_s_memrealtime();                        \
  } while (0)
#else
#define QNN_PHASE(k) \
  do {               \
  } while (0)
#endif

template <int GG, int GD>
__global__ __launch_bounds__(256) void k_int4_mlp(const MlpLaunch a) {
  extern __shared__ uint4 dyn_lds[];
  __shared__ float red[4][64];
  const int wave = dev::wave_id(), tid = threadIdx.x, lane = tid & 63, part = wave;
  const int wg = blockIdx.x;
  constexpr int QD = dev::scale_quads<GD>();
  constexpr int XG = 4 * (GG > GD ? GG : GD);
  const dev::XPlanes xs = dev::xplanes_at(dyn_lds, 1, XG);
  const I4Layout &lg = a.lg, &ld = a.ld;
  QNN_PHASE(0);

  // ---- gate/up item of this workgroup (qnn_int4.hip I4_SWIGLU, T = 1: units
  //      padded to 16 so the gate tile u and the up tile u + 8 share an XCD).
  const int units_gu = (2 * lg.blocks + 15) / 16 * 16;
  int unit = 0, slice = 0;
  const bool mapped = dev::map_tile(wg, a.slices_gu, units_gu, unit, slice);
  const int tile_m = 2 * ((unit >> 4) * 8 + (unit & 7)) + ((unit >> 3) & 1);
  const bool gu_on = mapped && tile_m < 2 * lg.blocks;
  const int tile = gu_on ? tile_m : 0;
  if (!gu_on) slice = 0;
  const int ws0 = slice * 4 * a.sps_gu, s0 = ws0 + part * a.sps_gu;
  const int ns = max(0, min(a.sps_gu, lg.steps - s0));
  const int sgroups = min(4 * a.sps_gu, lg.groups - ws0);

  // ---- down item (I4_STORE plan, per-op map) of this workgroup.
  int td = 0, sld = 0;
  const bool dn_on = wg < a.grid_dn && dev::map_tile(wg, a.slices_dn, ld.blocks, td, sld);
  if (!dn_on) td = sld = 0;
  const int wsd = sld * 4 * a.sps_dn, s0d = wsd + part * a.sps_dn;
  const int nsd = max(0, min(a.sps_dn, ld.steps - s0d));
  const int sgd = min(4 * a.sps_dn, ld.groups - wsd);

  // ---- 1) Loads: x slice and gate/up weights to registers.
  float4 xr[1][dev::x_iters<GG>()];
  uint4 w[GG];
  uint4 q[dev::scale_quads<GG>()];
  dev::load_x<1, GG>(xr, dev::rsrc(a.x, size_t(a.hidden) * 4), [](int) { return 0u; }, 1, ws0 * 32, sgroups * 32,
                     tid);
  dev::load_wq<GG>(w, q, dev::rsrc((tile & 1) ? a.unib : a.gnib, lg.nib_bytes()),
                   dev::rsrc((tile & 1) ? a.uscl : a.gscl, lg.scale_bytes()), lg, tile >> 1, s0, lane);
  float sc[GG];
  dev::pick_scales<GG>(sc, q, s0);  // after every load is issued

  // ---- 2) Gate/up item: stage x, integer dot, parts in LDS, split-K exchange;
  //         the last of the 2 x slices arrivals of a block writes its h rows and
  //         raises the block's flag.
  dev::stage_x<1, GG>(xs, xr, 1, ws0 * 32, sgroups * 32, a.hidden, tid, lane);
  __syncthreads();
  QNN_PHASE(1);
  float acc[1] = {0.0f};
  if (ns > 0) {
    dev::XPlanes xp = xs;
    const int g0 = part * a.sps_gu;
    xp.q = xs.q + size_t(g0) * dev::kXWords;
    xp.s2 = xs.s2 + g0;
    xp.off = xs.off + g0;
    dev::dot<1, GG>(acc, w, sc, xp, 1, 0, ns);
  }
  if (part > 0) red[part][lane] = acc[0];
  __syncthreads();
  QNN_PHASE(2);
  if (part == 0 && gu_on) {
    acc[0] += red[1][lane];
    acc[0] += red[2][lane];
    acc[0] += red[3][lane];
    dev::xstore(a.partial_gu + (size_t(tile) * a.slices_gu + slice) * 64 + lane, acc[0]);
    unsigned *ctr = &a.counters_gu[size_t(tile >> 1) * kCounterStride];
    if (dev::last_arrival(ctr, unsigned(2 * a.slices_gu), lane)) {
      const float *pt = a.partial_gu + size_t(tile & ~1) * a.slices_gu * 64 + lane;
      float gu[2];  // gate and up, their slices loaded in one batch
      dev::sum_slices<2, 16>(gu, [&](int s, int m) { return pt + size_t(m * a.slices_gu + s) * 64; }, a.slices_gu);
      QNN_PHASE(11);
      dev::reset_counter(ctr, lane);
      const int blk = tile >> 1, row = blk * 64 + lane;
      if (row < a.inter) dev::xstore(a.h + row, dev::silu(gu[0]) * gu[1]);
      __builtin_amdgcn_s_waitcnt(0);  // the block's h is at the coherence point
      if (lane == 0)
        __hip_atomic_store(a.flags + size_t(blk) * 64, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      QNN_PHASE(4);
    }
    QNN_PHASE(3);
  }
  if (!dn_on) return;

  // ---- Down weights to registers, issued only now, so that the gate/up
  //      weights of every workgroup are requested first and h is complete
  //      sooner.
  uint4 wd[GD];
  uint4 qd[QD];
  dev::load_wq<GD>(wd, qd, dev::rsrc(a.dnib, ld.nib_bytes()), dev::rsrc(a.dscl, ld.scale_bytes()), ld, td, s0d, lane);

  // ---- 3) Down item: wait for the blocks of h in its K-slice, stage them, dot
  //         with the weights already in registers, split-K exchange, y.
  __syncthreads();  // xs and red are reused
  if (wave == 0) {
    const int b0 = (wsd * 32) >> 6, nb = (sgd * 32 + 63) >> 6;  // h blocks of the slice (<= 64)
    unsigned spins = 0;
    for (;;) {
      const bool ready = lane >= nb || __hip_atomic_load(a.flags + size_t(b0 + lane) * 64, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
      if (__ballot(!ready) == 0) break;
      __builtin_amdgcn_s_sleep(1);
      if (++spins > (1u << 25)) {  // ~1 s: report and finish instead of hanging
        if (lane == 0) atomicOr(a.err, 2);
        break;
      }
    }
  }
  __syncthreads();
  QNN_PHASE(5);
  float4 hr[1][dev::x_iters<GD>()];
  dev::load_x<1, GD, dev::kCoherent>(hr, dev::rsrc(a.h, size_t(a.inter) * 4), [](int) { return 0u; }, 1, wsd * 32,
                                    sgd * 32, tid);
  dev::stage_x<1, GD>(xs, hr, 1, wsd * 32, sgd * 32, a.inter, tid, lane);
  __syncthreads();
  QNN_PHASE(6);
  float scd[GD];
  dev::pick_scales<GD>(scd, qd, s0d);
  acc[0] = 0.0f;
  if (nsd > 0) {
    dev::XPlanes xp = xs;
    const int g0 = part * a.sps_dn;
    xp.q = xs.q + size_t(g0) * dev::kXWords;
    xp.s2 = xs.s2 + g0;
    xp.off = xs.off + g0;
    dev::dot<1, GD>(acc, wd, scd, xp, 1, 0, nsd);
  }
  if (part > 0) red[part][lane] = acc[0];
  __syncthreads();
  QNN_PHASE(7);
  if (part > 0) return;
  acc[0] += red[1][lane];
  acc[0] += red[2][lane];
  acc[0] += red[3][lane];
  if (a.slices_dn > 1) {
    dev::xstore(a.partial_dn + (size_t(td) * a.slices_dn + sld) * 64 + lane, acc[0]);
    unsigned *ctr = &a.counters_dn[size_t(td) * kCounterStride];
    const bool last = dev::last_arrival(ctr, unsigned(a.slices_dn), lane);
    QNN_PHASE(9);
    if (!last) return;
    const float *pt = a.partial_dn + size_t(td) * a.slices_dn * 64 + lane;
    dev::sum_slices<1, 32>(acc, [&](int s, int) { return pt + size_t(s) * 64; }, a.slices_dn);
    QNN_PHASE(10);
    dev::reset_counter(ctr, lane);
  }
  const int row = td * 64 + lane;
  if (row < a.hidden) a.y[row] = acc[0];
  QNN_PHASE(8);
}

// An ordinary launch of at most the co-resident workgroup count (the caller
// checks it against mlp_capacity): on an otherwise idle device every
// workgroup is placed at once, and the bounded waits turn anything else into
// an error instead of a hang.  (A cooperative launch would guarantee the
// residency; it was measured slower.)
template <int GG, int GD>
bool launch_mlp(const MlpLaunch &a, int grid, hipStream_t st) {
  hipLaunchKernelGGL((k_int4_mlp<GG, GD>), dim3(grid), dim3(256), mlp_lds_bytes(GG, GD), st, a);
  return hipGetLastError() == hipSuccess;
}

template <int GG, int GD>
int capacity_of(int device) {
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&k_int4_mlp<GG, GD>), 256,
                                                   mlp_lds_bytes(GG, GD)) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return per_cu * cus;
}

}  // namespace

int mlp_phase_read(void *dst, size_t bytes) {
#ifdef QNN_PHASE_TRACE
  const size_t n = std::min(bytes, sizeof(g_phase));
  if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_phase), n, 0, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  static const unsigned long long zeros[kPhaseWGs * kPhases] = {};
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_phase), zeros, sizeof(g_phase), 0, hipMemcpyHostToDevice) != hipSuccess) return -1;
  return int(n / 8);
#else
  (void)dst;
  (void)bytes;
  return -2;
#endif
}

size_t mlp_lds_bytes(int gg, int gd) { return dev::xplanes_bytes(1, 4 * std::max(gg, gd)); }

int mlp_capacity(int gg, int gd, int device) {
  if (gg == 4 && gd == 4) return capacity_of<4, 4>(device);
  if (gg == 2 && gd == 2) return capacity_of<2, 2>(device);
  if (gg == 2 && gd == 4) return capacity_of<2, 4>(device);
  if (gg == 4 && gd == 2) return capacity_of<4, 2>(device);
  if (gg == 8 && gd == 4) return capacity_of<8, 4>(device);
  if (gg == 4 && gd == 8) return capacity_of<4, 8>(device);
  if (gg == 8 && gd == 8) return capacity_of<8, 8>(device);
  return 0;
}

bool mlp_launch(const MlpLaunch &a, int gg, int gd, int grid, hipStream_t st) {
  if (gg == 4 && gd == 4) return launch_mlp<4, 4>(a, grid, st);
  if (gg == 2 && gd == 2) return launch_mlp<2, 2>(a, grid, st);
  if (gg == 2 && gd == 4) return launch_mlp<2, 4>(a, grid, st);
  if (gg == 4 && gd == 2) return launch_mlp<4, 2>(a, grid, st);
  if (gg == 8 && gd == 4) return launch_mlp<8, 4>(a, grid, st);
  if (gg == 4 && gd == 8) return launch_mlp<4, 8>(a, grid, st);
  if (gg == 8 && gd == 8) return launch_mlp<8, 8>(a, grid, st);
  return false;
}

}  // namespace qnn
