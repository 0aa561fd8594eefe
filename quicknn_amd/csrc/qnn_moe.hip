// qnn_moe.hip -- routed experts on the device (native INT4 experts).
//
// Replaces the host orchestration of TLLMMoE.forward
// (src/models/QuickNN.Models.LLM.MoE.pas:376-448): there the route ids are
// read back to the host, counted per expert, and every routed expert is run
// as its own gate/up SwiGLU (op 68 / ops 56+SWIGLU) and down projection,
// accumulated as out += p * y in ascending expert id (op 69 for one token,
// GO_MOE_SCATTER otherwise, moe.comp:70 and :125-126).
//
// Here the routes stay on the GPU and a layer's experts take two launches:
//   1. gate/up: h[R] = silu(W_g[e] x_t) * (W_u[e] x_t) for every route
//      position R = t*topk + j (token t, expert e = id[R]);
//   2. down:    y[R] = W_d[e] h[R], then out[t] = sum over the token's routes in
//      ascending expert id of p[R] * y[R] (starting from 0, the reference's
//      GO_FILL + accumulate order).
// The grid is (4 tiles, slot, K-slice); slot s is the s-th smallest expert id
// present in the routes, so only routed experts' weights are read, each once
// per launch for all of its tokens.  Every workgroup derives its slot's expert
// and token positions from the route ids itself (a few LDS operations), so no
// planning launch or host readback is needed.  Split-K slices of a
// (slot, tile) are combined by the last to finish, and in the down launch the
// last (slot, tile) of a tile to finish combines the experts, both in a fixed
// order, so results do not depend on timing.
#include "qnn_int4_dev.h"

namespace qnn {
namespace {

constexpr int kMaxPos = 128;  // positions per expert (= tokens, since a token's route ids are distinct)

struct MoEPlan {
  uint32_t mask[kMoEMaxExperts / 32];
  int e, c, active;
  int pos[kMaxPos];
  uint32_t ids[kMoEMaxRoutes];
  uint8_t ord[kMoEMaxRoutes];
};

// Wave 0 builds the plan of `slot` in LDS; the caller synchronises.
__device__ void build_plan(MoEPlan &pl, const MoELaunch &a, int n, int slot, int lane) {
  if (lane < kMoEMaxExperts / 32) pl.mask[lane] = 0u;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  bool bad = false;
  for (int i = lane; i < n; i += 64) {
    const uint32_t id = __float_as_uint(a.routes[i]);
    pl.ids[i] = id;
    if (id < uint32_t(a.experts)) atomicOr(&pl.mask[id >> 5], 1u << (id & 31));
    else bad = true;
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // slot -> expert: the (slot)-th set bit of the mask
  const uint32_t word = lane < kMoEMaxExperts / 32 ? pl.mask[lane] : 0u;
  const int cnt = __popc(word);
  int incl = cnt;
#pragma unroll
  for (int d = 1; d < kMoEMaxExperts / 32; d <<= 1) {
    const int t = __shfl_up(incl, d);
    if (lane >= d) incl += t;
  }
  const int active = __shfl(incl, kMoEMaxExperts / 32 - 1);
  const int excl = incl - cnt;
  int e = -1;
  if (lane < kMoEMaxExperts / 32 && slot >= excl && slot < incl) {
    uint32_t wv = word;
    for (int j = excl; j < slot; ++j) wv &= wv - 1u;
    e = lane * 32 + __ffs(wv) - 1;
  }
  const uint64_t has = __ballot(e >= 0);
  e = has ? __shfl(e, __ffsll((unsigned long long)has) - 1) : -1;
  // positions routed to e, ascending
  int c = 0;
  if (e >= 0) {
    for (int i0 = 0; i0 < n; i0 += 64) {
      const int i = i0 + lane;
      const bool hit = i < n && pl.ids[i] == uint32_t(e);
      const uint64_t bm = __ballot(hit);
      if (hit) {
        const int r = c + __popcll(bm & ((1ull << lane) - 1ull));
        if (r < kMaxPos) pl.pos[r] = i;
      }
      c += __popcll(bm);
    }
  }
  const bool any_bad = __ballot(bad) != 0;
  if (lane == 0) {
    pl.e = e;
    pl.c = min(c, min(a.rows, kMaxPos));
    pl.active = active;
    if (any_bad || c > a.rows) atomicOr(a.err, 8);  // invalid expert id / an expert twice in one token
  }
}

// ord[t*k + r] = j of token t's r-th smallest route id (ties: lower j), by
// wave 0 of every down-launch workgroup (only a tile's last arrival reads it).
__device__ void build_order(MoEPlan &pl, int n, int k, int lane) {
  for (int i = lane; i < n; i += 64) {
    const int t0 = (i / k) * k;
    const uint32_t id = pl.ids[i];
    int r = 0;
    for (int j = 0; j < k; ++j) {
      const uint32_t o = pl.ids[t0 + j];
      r += (o < id) || (o == id && t0 + j < i);
    }
    pl.ord[t0 + r] = uint8_t(i - t0);
  }
}

// DOWN = false: gate/up launch (a tile is half a 64-lane block: its gate rows
// in lanes 0-31 and the same up rows in lanes 32-63).  DOWN = true: down
// launch (a tile is one block) + expert combine.  A workgroup is one tile of
// one slot and a K-slice of 4*sps steps; wave w takes steps [w*sps, (w+1)*sps)
// of it and the four partial sums meet in LDS in wave order.
template <int MT, int GSW, bool DOWN>
__global__ __launch_bounds__(256) void k_moe(const MoELaunch a, const int slices, const int sps, const int slots) {
  extern __shared__ uint4 dyn_lds[];
  __shared__ float red[3][MT][64];
  const int n = a.rows * a.topk;
  const I4Layout &l = DOWN ? a.dn : a.gu;
  const int tiles = DOWN ? l.blocks : 2 * l.blocks;
  const int nout = DOWN ? a.hidden : a.inter;
  int tile, rest;
  if (!dev::map_tile(blockIdx.x, slots * slices, tiles, tile, rest)) return;
  const int slot = rest / slices, slice = rest - slot * slices;
  const int tid = threadIdx.x, lane = tid & 63, wave = dev::wave_id();

  __shared__ MoEPlan pl;
  if (wave == 0) {
    build_plan(pl, a, n, slot, lane);
    if (DOWN) build_order(pl, n, a.topk, lane);
  }
  __syncthreads();
  const int e = pl.e, c = pl.c;
  if (e < 0) return;  // fewer routed experts than slots

  const int L = l.lanes, j = lane & (L - 1);
  const int ws0 = slice * 4 * sps;                         // first step of the slice
  const int s0 = ws0 + wave * sps;                         // first step of this wave
  const int ns = max(0, min(sps, l.steps - s0));
  const int sgroups = min(4 * sps * L, l.groups - ws0 * L);
  const int kin = DOWN ? a.inter : a.hidden;  // both multiples of 4 (checked by the host)

  // weights of expert e: one contiguous matrix per expert; gate/up lanes
  // 32-63 read the up matrix, which follows the gate matrix, through the same
  // (workgroup-uniform) resources at a per-lane offset
  int b = tile, wl = lane;
  const uint8_t *wbase;
  size_t wbytes;
  uint32_t moff = 0;
  if (DOWN) {
    wbase = a.down + size_t(e) * a.dn_stride;
    wbytes = a.dn_stride;
  } else {
    b = tile >> 1;
    wl = (tile & 1) * 32 + (lane & 31);
    wbase = a.gate_up + size_t(2 * e) * a.gu_stride;
    wbytes = 2 * a.gu_stride;
    moff = lane < 32 ? 0u : uint32_t(a.gu_stride);
  }
  // activation rows: h[R] (down) or x[token of R] (gate/up)
  const dev::Rsrc xsrc = DOWN ? dev::rsrc(a.h, size_t(n) * a.inter * 4) : dev::rsrc(a.x, size_t(a.rows) * a.hidden * 4);
  auto xoff = [&](int m) -> uint32_t {
    const int R = pl.pos[min(m, c - 1)];
    return DOWN ? uint32_t(R) * uint32_t(a.inter) * 4u : uint32_t(R / a.topk) * uint32_t(a.hidden) * 4u;
  };
  float4 xr[MT][dev::x_iters<GSW>()];
  dev::load_x<MT, GSW>(xr, xsrc, xoff, min(c, MT), ws0 * L * 32, sgroups * 32, tid);
  uint4 w[GSW];
  float sc[GSW];
  dev::load_w<GSW>(w, sc, dev::rsrc(wbase, wbytes), dev::rsrc(wbase + l.nib_bytes(), wbytes - l.nib_bytes()), l, b, s0,
                   wl, moff, moff);

  const dev::XPlanes xs = dev::xplanes_at(dyn_lds, MT, 4 * sps * L);
  dev::XPlanes xw = xs;  // this wave's groups
  xw.q = xs.q + size_t(wave) * sps * L * dev::kXWords;
  xw.s2 = xs.s2 + wave * sps * L;
  xw.off = xs.off + wave * sps * L;
  float *part = a.partial + (size_t(tile) * slices + slice) * n * 64 + lane;
  const int row = DOWN ? b * l.rpb + lane / L : b * l.rpb + wl / L;
  auto finish = [&](int R, float v) {  // final value of this lane's row for position R
    if (DOWN) {
      if (j == 0 && row < nout) dev::xstore(a.y + size_t(R) * a.hidden + row, v, a.xcd_local);
    } else {
      const float u = __shfl_down(v, 32);
      if (lane < 32 && j == 0 && row < nout) a.h[size_t(R) * a.inter + row] = dev::silu(v) * u;
    }
  };

  for (int m0 = 0; m0 < c; m0 += MT) {
    if (m0 > 0) {
      dev::load_x<MT, GSW>(xr, xsrc, [&](int m) { return xoff(m0 + m); }, min(c - m0, MT), ws0 * L * 32, sgroups * 32,
                           tid);
      __syncthreads();  // the previous chunk's LDS reads are done
    }
    dev::stage_x<MT, GSW>(xs, xr, min(c - m0, MT), ws0 * L * 32, sgroups * 32, kin, tid, lane);
    __syncthreads();
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    if (ns > 0) {
      dev::dot<MT, GSW>(acc, w, sc, xw, L, j, ns);
      dev::reduce_lanes<MT>(acc, L);
    }
    if (wave > 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m) red[wave - 1][m][lane] = acc[m];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        acc[m] = ((acc[m] + red[0][m][lane]) + red[1][m][lane]) + red[2][m][lane];
        if (m0 + m < c) {
          const int R = pl.pos[m0 + m];
          if (slices > 1) dev::xstore(part + size_t(R) * 64, acc[m], a.xcd_local);
          else finish(R, acc[m]);
        }
      }
    }
  }
  if (wave > 0) return;

  // split-K: the last slice of (slot, tile) sums the slices in order
  if (slices > 1) {
    dev::check_xcd(a.xcd_local, a.err, lane);
    unsigned *ctr = &a.counters[(size_t(tile) * slots + slot) * kCounterStride];
    if (!dev::last_arrival(ctr, unsigned(slices), lane)) return;
    const float *pt = a.partial + size_t(tile) * slices * n * 64 + lane;
    for (int m0 = 0; m0 < c; m0 += MT) {
      float acc[MT];
      dev::sum_slices<MT, 4>(
          acc, [&](int s, int m) { return pt + (size_t(s) * n + pl.pos[min(m0 + m, c - 1)]) * 64; }, slices,
          a.xcd_local);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m0 + m < c) finish(pl.pos[m0 + m], acc[m]);
    }
    dev::reset_counter(ctr, lane);
  }
  if (!DOWN) return;

  // expert combine: the last (slot, tile) of this tile to finish; lane (r, j)
  // combines row r for tokens j, j+L, ...
  dev::check_xcd(a.xcd_local, a.err, lane);
  unsigned *cctr = &a.counters[(size_t(tiles) * slots + tile) * kCounterStride];
  if (!dev::last_arrival(cctr, unsigned(pl.active), lane)) return;
  if (row < nout) {
    for (int tk = j; tk < a.rows; tk += L) {
      float acc = 0.0f;
      for (int r = 0; r < a.topk; ++r) {
        const int R = tk * a.topk + pl.ord[tk * a.topk + r];
        if (pl.ids[R] >= uint32_t(a.experts)) continue;
        const float p = a.routes[n + R];
        const float v = dev::xload(a.y + size_t(R) * a.hidden + row, a.xcd_local);
        acc = add_mul_nofma(acc, v, p);  // moe.comp:70 / :126: out + y*p
      }
      a.out[size_t(tk) * a.hidden + row] = acc;
    }
  }
  dev::reset_counter(cctr, lane);
}

template <int MT, int GSW>
void launch_mt(const MoELaunch &a, const MoEPlanSizes &p, hipStream_t s) {
  const int tgu = 2 * a.gu.blocks, tdn = a.dn.blocks;
  const int ggu = (tgu + 7) / 8 * 8 * p.slots * p.slices_gu;
  const int gdn = (tdn + 7) / 8 * 8 * p.slots * p.slices_dn;
  hipLaunchKernelGGL((k_moe<MT, GSW, false>), dim3(ggu), dim3(256), p.lds_gu, s, a, p.slices_gu, p.sps_gu, p.slots);
  hipLaunchKernelGGL((k_moe<MT, GSW, true>), dim3(gdn), dim3(256), p.lds_dn, s, a, p.slices_dn, p.sps_dn, p.slots);
}

}  // namespace

MoEPlanSizes moe_plan(const MoELaunch &a) {
  MoEPlanSizes p;
  const int n = a.rows * a.topk;
  p.slots = std::min(a.experts, n);
  p.mt = a.rows == 1 ? 1 : (a.rows * a.topk <= 2 * a.experts ? 2 : 4);
  // Steps per wave: 2 (a workgroup slice of 8 groups per 64-row tile),
  // measured fastest at 1 and 16 tokens for 128 experts of 768 x 2048;
  // QNN_MOE_SPS overrides.  Bounded by the activation-slice LDS budget.
  const int forced = env_int("QNN_MOE_SPS", 0);
  auto steps = [&](const I4Layout &l, int) {
    const int lds_cap = int((48 << 10) / (size_t(p.mt) * 4 * l.lanes * (dev::kXWords * 4 + 8)));
    const int cap = std::max(1, std::min(8, lds_cap));
    return std::min(forced > 0 ? forced : 2, cap);
  };
  p.sps_gu = steps(a.gu, 2 * a.gu.blocks);
  p.sps_dn = steps(a.dn, a.dn.blocks);
  p.slices_gu = (a.gu.steps + 4 * p.sps_gu - 1) / (4 * p.sps_gu);
  p.slices_dn = (a.dn.steps + 4 * p.sps_dn - 1) / (4 * p.sps_dn);
  const int need = std::max(p.sps_gu, p.sps_dn);
  p.gsw = need <= 1 ? 1 : (need <= 2 ? 2 : (need <= 4 ? 4 : 8));
  p.lds_gu = dev::xplanes_bytes(p.mt, 4 * p.sps_gu * a.gu.lanes);
  p.lds_dn = dev::xplanes_bytes(p.mt, 4 * p.sps_dn * a.dn.lanes);
  const int tgu = 2 * a.gu.blocks, tdn = a.dn.blocks;
  p.partial_floats = std::max(size_t(tgu) * p.slices_gu, size_t(tdn) * p.slices_dn) * n * 64;
  p.counters = (size_t(std::max(tgu, tdn)) * p.slots + tdn) * kCounterStride;
  return p;
}

void moe_launch(const MoELaunch &a, const MoEPlanSizes &p, hipStream_t s) {
  switch (p.mt * 16 + p.gsw) {
    case 1 * 16 + 1: launch_mt<1, 1>(a, p, s); break;
    case 1 * 16 + 2: launch_mt<1, 2>(a, p, s); break;
    case 1 * 16 + 4: launch_mt<1, 4>(a, p, s); break;
    case 1 * 16 + 8: launch_mt<1, 8>(a, p, s); break;
    case 2 * 16 + 1: launch_mt<2, 1>(a, p, s); break;
    case 2 * 16 + 2: launch_mt<2, 2>(a, p, s); break;
    case 2 * 16 + 4: launch_mt<2, 4>(a, p, s); break;
    case 2 * 16 + 8: launch_mt<2, 8>(a, p, s); break;
    case 4 * 16 + 1: launch_mt<4, 1>(a, p, s); break;
    case 4 * 16 + 2: launch_mt<4, 2>(a, p, s); break;
    case 4 * 16 + 4: launch_mt<4, 4>(a, p, s); break;
    case 4 * 16 + 8: launch_mt<4, 8>(a, p, s); break;
    default: fail(QNN_E_INVALID_OP, "MoE launch plan");
  }
  hip_check(hipGetLastError(), "moe launch");
}

}  // namespace qnn
