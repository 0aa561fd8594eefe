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
// The grid is (tile, slot, K-slice); slot s is the s-th smallest expert id
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

// Wave 0 of the combining workgroup: ord[t*k + r] = j of the token's r-th
// smallest route id (ties: lower j).
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
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// DOWN = false: gate/up launch (tile = 32 output rows, lanes 0-31 gate, 32-63
// up).  DOWN = true: down launch (tile = 64 rows) + expert combine.
template <int MT, int GSW, bool DOWN>
__global__ __launch_bounds__(256) void k_moe(const MoELaunch a, const int slices, const int slots) {
  constexpr int GS = 4 * GSW;
  const int n = a.rows * a.topk;
  const I4Layout &L = DOWN ? a.dn : a.gu;
  const int tiles = DOWN ? a.dn.tiles : (a.inter + 31) / 32;
  const int nout = DOWN ? a.hidden : a.inter;
  int tile, rest;
  if (!dev::map_tile(blockIdx.x, slots * slices, tiles, tile, rest)) return;
  const int slot = rest / slices, slice = rest - slot * slices;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  __shared__ MoEPlan pl;
  if (wave == 0) build_plan(pl, a, n, slot, lane);
  __syncthreads();
  const int e = pl.e, c = pl.c;
  if (e < 0) return;  // fewer routed experts than slots

  const int g0 = slice * GS;
  const int ng = min(GS, L.g4 - g0);
  const int gw0 = wave * GSW;
  const int ngw = max(0, min(GSW, ng - gw0));
  const int gq0 = g0 + gw0;

  // weights of expert e: one contiguous tiled matrix per expert
  int stile = tile, srow = lane;
  const uint8_t *wbase;
  if (DOWN) {
    wbase = a.down + size_t(e) * a.dn_stride;
  } else {
    stile = tile >> 1;
    srow = (tile & 1) * 32 + (lane & 31);
    wbase = (lane < 32 ? a.gate : a.up) + size_t(e) * a.gu_stride;
  }
  const uint4 *nib = reinterpret_cast<const uint4 *>(wbase) + (size_t(stile) * L.g4 + gq0) * 64 + srow;
  const float *scl =
      reinterpret_cast<const float *>(wbase + L.nib_bytes()) + (size_t(stile) * (L.g4 >> 2) + (gq0 >> 2)) * 256 + srow * 4;
  const int kin = DOWN ? a.inter : a.hidden;
  auto xrow = [&](int m) -> const float * {
    if (m >= c) return nullptr;
    const int R = pl.pos[m];
    return DOWN ? a.h + size_t(R) * a.inter : a.x + size_t(R / a.topk) * a.hidden;
  };
  const bool vec4 = (kin % 4) == 0;

  float4 xr[MT][dev::x_iters<GS>()];
  dev::load_x<MT, GS>(xr, xrow, g0, ng, kin, vec4, tid);
  uint4 w[GSW];
  float sc[GSW];
  dev::load_w<GSW>(w, sc, nib, scl, gq0, ngw);

  __shared__ dev::XTile<MT, GS> xs;
  __shared__ float red[3][MT][64];
  float *part = a.partial + (size_t(tile) * slices + slice) * n * 64 + lane;
  auto finish = [&](int R, float v) {  // final value of row (tile, lane) for position R
    if (DOWN) {
      const int row = tile * 64 + lane;
      if (row < nout) dev::xstore(a.y + size_t(R) * a.hidden + row, v, a.xcd_local);
    } else {
      const float u = __shfl_down(v, 32);
      const int row = tile * 32 + lane;
      if (lane < 32 && row < nout) a.h[size_t(R) * a.inter + row] = dev::silu(v) * u;
    }
  };

  for (int m0 = 0; m0 < c; m0 += MT) {
    if (m0 > 0) {
      auto xrow_c = [&](int m) { return xrow(m0 + m); };
      dev::load_x<MT, GS>(xr, xrow_c, g0, ng, kin, vec4, tid);
      __syncthreads();  // the previous chunk's LDS reads are done
    }
    dev::stage_x<MT, GS>(xs, xr, tid, lane);
    __syncthreads();
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    dev::dot<MT, GS, GSW>(acc, w, sc, xs, gw0, ngw);
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
          acc,
          [&](int s, int m) { return pt + (size_t(s) * n + pl.pos[min(m0 + m, c - 1)]) * 64; }, slices,
          a.xcd_local);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (m0 + m < c) finish(pl.pos[m0 + m], acc[m]);
    }
    dev::reset_counter(ctr, lane);
  }
  if (!DOWN) return;

  // expert combine: the last (slot, tile) of this tile to finish
  dev::check_xcd(a.xcd_local, a.err, lane);
  unsigned *cctr = &a.counters[(size_t(tiles) * slots + tile) * kCounterStride];
  if (!dev::last_arrival(cctr, unsigned(pl.active), lane)) return;
  build_order(pl, n, a.topk, lane);
  const int row = tile * 64 + lane;
  for (int t = 0; t < a.rows; ++t) {
    float acc = 0.0f;
    for (int r = 0; r < a.topk; ++r) {
      const int R = t * a.topk + pl.ord[t * a.topk + r];
      if (pl.ids[R] >= uint32_t(a.experts)) continue;
      const float p = a.routes[n + R];
      const float v = row < nout ? dev::xload(a.y + size_t(R) * a.hidden + row, a.xcd_local) : 0.0f;
      acc = add_mul_nofma(acc, v, p);  // moe.comp:70 / :126: out + y*p
    }
    if (row < nout) a.out[size_t(t) * a.hidden + row] = acc;
  }
  dev::reset_counter(cctr, lane);
}

template <int MT, int GSW>
void launch_mt(const MoELaunch &a, int slices_gu, int slices_dn, int slots, hipStream_t s) {
  const int tgu = (a.inter + 31) / 32, tdn = a.dn.tiles;
  const int ggu = (tgu + 7) / 8 * 8 * slots * slices_gu;
  const int gdn = (tdn + 7) / 8 * 8 * slots * slices_dn;
  hipLaunchKernelGGL((k_moe<MT, GSW, false>), dim3(ggu), dim3(256), 0, s, a, slices_gu, slots);
  hipLaunchKernelGGL((k_moe<MT, GSW, true>), dim3(gdn), dim3(256), 0, s, a, slices_dn, slots);
}

}  // namespace

MoEPlanSizes moe_plan(const MoELaunch &a) {
  MoEPlanSizes p;
  const int n = a.rows * a.topk;
  p.slots = std::min(a.experts, n);
  p.mt = a.rows == 1 ? 1 : (a.rows * a.topk <= 2 * a.experts ? 2 : 4);
  p.gsw = env_int("QNN_MOE_GSW", 0);
  if (p.gsw != 1 && p.gsw != 2 && p.gsw != 4) {
    // largest slice whose group count divides both matrices' groups evenly
    p.gsw = 1;
    for (int g : {4, 2}) {
      if (a.gu.g4 % (4 * g) == 0 && a.dn.g4 % (4 * g) == 0) { p.gsw = g; break; }
    }
  }
  const int gs = 4 * p.gsw;
  p.slices_gu = (a.gu.g4 + gs - 1) / gs;
  p.slices_dn = (a.dn.g4 + gs - 1) / gs;
  const int tgu = (a.inter + 31) / 32, tdn = a.dn.tiles;
  p.partial_floats = std::max(size_t(tgu) * p.slices_gu, size_t(tdn) * p.slices_dn) * n * 64;
  p.counters = (size_t(std::max(tgu, tdn)) * p.slots + tdn) * kCounterStride;
  return p;
}

void moe_launch(const MoELaunch &a, const MoEPlanSizes &p, hipStream_t s) {
  switch (p.mt * 16 + p.gsw) {
    case 1 * 16 + 1: launch_mt<1, 1>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 1 * 16 + 2: launch_mt<1, 2>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 1 * 16 + 4: launch_mt<1, 4>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 2 * 16 + 1: launch_mt<2, 1>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 2 * 16 + 2: launch_mt<2, 2>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 2 * 16 + 4: launch_mt<2, 4>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 4 * 16 + 1: launch_mt<4, 1>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 4 * 16 + 2: launch_mt<4, 2>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    case 4 * 16 + 4: launch_mt<4, 4>(a, p.slices_gu, p.slices_dn, p.slots, s); break;
    default: fail(QNN_E_INVALID_OP, "MoE launch plan");
  }
  hip_check(hipGetLastError(), "moe launch");
}

}  // namespace qnn
