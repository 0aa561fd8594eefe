// qnn_moe.hip -- routed experts on the device (native INT4 experts).
//
// Replaces the host orchestration of TLLMMoE.forward
// (src/models/QuickNN.Models.LLM.MoE.pas:376-448): there the route ids are
// read back to the host, counted per expert, and every routed expert is run
// as its own gate/up SwiGLU (op 68 / ops 56+SWIGLU) and down projection,
// accumulated as out += p * y in ascending expert id (op 69 for one token,
// GO_MOE_SCATTER otherwise, moe.comp:70 and :125-126).
//
// Here the routes stay on the GPU and a layer's experts take two launches
// after a small planning launch:
//   0. plan:    per slot, its expert and the route positions routed to it
//      (k_moe_plan, from the route ids; no host readback);
//   1. gate/up: h[R] = silu(W_g[e] x_t) * (W_u[e] x_t) for every route
//      position R = t*topk + j (token t, expert e = id[R]);
//   2. down:    y[R] = W_d[e] h[R], then out[t] = sum over the token's routes in
//      ascending expert id of p[R] * y[R] (starting from 0, the reference's
//      GO_FILL + accumulate order).
// The grid is (4 tiles, slot, K-slice); slot s is the s-th smallest expert id
// present in the routes, so only routed experts' weights are read, each once
// per launch for all of its tokens.  Split-K slices of a
// (slot, tile) are combined by the last to finish, and in the down launch the
// last (slot, tile) of a tile to finish combines the experts, both in a fixed
// order, so results do not depend on timing.
#include "qnn_int4_dev.h"
#include "qnn_route_dev.h"

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
  for (int i0 = 0; i0 < n; i0 += 256) {  // 4 route ids per lane in flight together
    uint32_t idv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) idv[r] = __float_as_uint(a.routes[min(i0 + r * 64 + lane, n - 1)]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + r * 64 + lane;
      if (i < n) {
        pl.ids[i] = idv[r];
        if (idv[r] < uint32_t(a.experts)) atomicOr(&pl.mask[idv[r] >> 5], 1u << (idv[r] & 31));
        else bad = true;
      }
    }
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

// Multi-token launches: every slot's plan is built once per call by
// k_moe_plan (the same build_plan / build_order that each workgroup ran
// itself before) and stored as a record per slot -- expert, position count,
// active experts, positions -- followed by the route ids and the per-token
// order.  A k_moe workgroup then loads its slot's record in one batch of
// loads instead of rebuilding the plan (batch 16: building it twice per
// workgroup cost 16 us per layer).
constexpr int kSlotWords = 4 + kMaxPos;
// Workgroups 0 .. slots-1 build one slot's record each; the last one (slot
// == slots) writes the route ids and the per-token order, in parallel with
// them.
__global__ __launch_bounds__(64) void k_moe_plan(const MoELaunch a, const int slots) {
  __shared__ MoEPlan pl;
  const int n = a.rows * a.topk, slot = blockIdx.x, lane = threadIdx.x;
  if (slot == slots) {
    for (int i = lane; i < n; i += 64) pl.ids[i] = __float_as_uint(a.routes[i]);
    dev::wave_lds_sync();
    build_order(pl, n, a.topk, lane);
    dev::wave_lds_sync();
    int *ids = a.plan + size_t(slots) * kSlotWords;
    for (int i = lane; i < n; i += 64) {
      ids[i] = int(pl.ids[i]);
      ids[n + i] = int(pl.ord[i]);
    }
    return;
  }
  build_plan(pl, a, n, slot, lane);
  dev::wave_lds_sync();
  int *rec = a.plan + size_t(slot) * kSlotWords;
  if (lane == 0) {
    rec[0] = pl.e;
    rec[1] = pl.c;
    rec[2] = pl.active;
    rec[3] = 0;
  }
  for (int i = lane; i < kMaxPos; i += 64) rec[4 + i] = i < pl.c ? pl.pos[i] : 0;
}
// Wave 0 loads `slot`'s plan record (and, with IDS, the route ids and the
// order) into LDS; the caller synchronises.
template <bool IDS>
__device__ void load_plan(MoEPlan &pl, const MoELaunch &a, int n, int slot, int slots, int lane) {
  const int *rec = a.plan + size_t(slot) * kSlotWords;
  const int r0 = rec[lane], r1 = rec[64 + lane], r2 = rec[128 + min(lane, kSlotWords - 129)];
  const int c = __shfl(r0, 1), active = __shfl(r0, 2);
  if (lane == 0) {
    pl.e = r0;
    pl.c = c;
    pl.active = active;
  }
  if (lane >= 4) pl.pos[lane - 4] = r0;
  pl.pos[60 + lane] = r1;
  if (lane < kSlotWords - 128) pl.pos[124 + lane] = r2;
  if (IDS) {
    const int *ids = a.plan + size_t(slots) * kSlotWords;
    for (int i0 = 0; i0 < n; i0 += 256) {  // 4 ids and orders per lane in flight together
      int iv[4], ov[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = min(i0 + r * 64 + lane, n - 1);
        iv[r] = ids[i];
        ov[r] = ids[n + i];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i0 + r * 64 + lane;
        if (i < n) {
          pl.ids[i] = uint32_t(iv[r]);
          pl.ord[i] = uint8_t(ov[r]);
        }
      }
    }
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
  // Expert layouts have one lane per row (int4_layout(.., true)), so a
  // slice is at most 4 x 8 x 32 elements: one pass of activation loads
  // (x_iters<2>), 12 fewer VGPRs than the lanes-per-row general form.
  constexpr int XG = GSW <= 8 ? 2 : GSW;
  const int n = a.rows * a.topk;
  const I4Layout &l = DOWN ? a.dn : a.gu;
  const int tiles = DOWN ? l.blocks : 2 * l.blocks;
  const int nout = DOWN ? a.hidden : a.inter;
  int tile, rest;
  if (!dev::map_tile(blockIdx.x, slots * slices, tiles, tile, rest)) return;
  const int slot = rest / slices, slice = rest - slot * slices;
  const int tid = threadIdx.x, lane = tid & 63, wave = dev::wave_id();

  __shared__ MoEPlan pl;
  if (wave == 0) load_plan<DOWN>(pl, a, n, slot, slots, lane);
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
  float4 xr[MT][dev::x_iters<XG>()];
  dev::load_x<MT, XG>(xr, xsrc, xoff, min(c, MT), ws0 * L * 32, sgroups * 32, tid);
  const dev::XPlanes xs = dev::xplanes_at(dyn_lds, MT, 4 * sps * L);
  // The first chunk's activations are requested, then the weights, then the
  // activations are staged (waiting for them alone).  With the plan loaded
  // rather than built this order is the fastest (batch 16: 92.5 -> 89.6 us
  // against staging before the weight loads are issued; weights first:
  // 92.1 us).
  uint4 w[GSW];
  float sc[GSW];
  // Down: resources that end with this block (K = 768 is 24 steps, so the
  // fourth wave of an 8-step slice has none and reads zeros instead of the
  // next block's weights; down traffic was 1.38x the weight bytes).  Gate/up:
  // both matrices through one resource at a per-lane offset, whose K-slices
  // cover the steps exactly at the shapes measured.
  if (DOWN)
    dev::load_w<GSW>(w, sc, dev::block_nib_rsrc(wbase, l, b), dev::block_scl_rsrc(wbase + l.nib_bytes(), l, b), l, b, s0,
                     wl);
  else
    dev::load_w<GSW>(w, sc, dev::rsrc(wbase, wbytes), dev::rsrc(wbase + l.nib_bytes(), wbytes - l.nib_bytes()), l, b,
                     s0, wl, moff, moff);
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the staging waits for x
  dev::stage_x<MT, XG>(xs, xr, min(c, MT), ws0 * L * 32, sgroups * 32, kin, tid, lane);

  dev::XPlanes xw = xs;  // this wave's groups
  xw.q = xs.q + size_t(wave) * sps * L * dev::kXWords;
  xw.s2 = xs.s2 + wave * sps * L;
  xw.off = xs.off + wave * sps * L;
  float *part = a.partial + (size_t(tile) * slices + slice) * n * 64 + lane;
  const int row = DOWN ? b * l.rpb + lane / L : b * l.rpb + wl / L;
  auto finish = [&](int R, float v) {  // final value of this lane's row for position R
    if (DOWN) {
      if (j == 0 && row < nout) dev::xstore(a.y + size_t(R) * a.hidden + row, v);
    } else {
      const float u = dev::xor_lanes<32>(v);  // lanes 0-31 take 32-63
      if (lane < 32 && j == 0 && row < nout) a.h[size_t(R) * a.inter + row] = dev::silu(v) * u;
    }
  };

  for (int m0 = 0; m0 < c; m0 += MT) {
    if (m0 > 0) {
      __syncthreads();  // the previous chunk's LDS reads are done
      dev::stage_x<MT, XG>(xs, xr, min(c - m0, MT), ws0 * L * 32, sgroups * 32, kin, tid, lane);
    }
    __syncthreads();
    // The next chunk's activations are requested now (its staging is done
    // with these registers), so their latency overlaps this chunk's products
    // and part sums instead of following them (batch 16: 101.5 -> 100.9 us).
    if (m0 + MT < c)
      dev::load_x<MT, XG>(xr, xsrc, [&](int m) { return xoff(m0 + MT + m); }, min(c - m0 - MT, MT), ws0 * L * 32,
                           sgroups * 32, tid);
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    if (ns > 0) {
      // The weights are unpacked inside every token pass: hoisted out of the
      // pass loop (the compiler's choice) the unpacked nibbles of all steps
      // stayed live, 138 VGPRs and three workgroups per CU; unpacked per pass
      // 114 VGPRs and four (batch 16: 85.9 -> 79.8 us; most experts have one
      // token, so one pass).
#pragma unroll
      for (int g = 0; g < GSW; ++g) asm volatile("" : "+v"(w[g].x), "+v"(w[g].y), "+v"(w[g].z), "+v"(w[g].w));
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
          if (slices > 1) dev::xstore(part + size_t(R) * 64, acc[m]);
          else finish(R, acc[m]);
        }
      }
    }
  }
  if (!DOWN && wave > 0) return;

  // split-K: the last slice of (slot, tile) sums the slices in order.  Down
  // launch: the last (slot, tile) of a tile to finish then owns that tile's
  // expert combine, which all four waves share.
  __shared__ int owner;
  if (wave == 0) {
    bool last = true;
    if (slices > 1) {
      unsigned *ctr = &a.counters[(size_t(tile) * slots + slot) * kCounterStride];
      last = dev::last_arrival(ctr, unsigned(slices), lane);
      if (last) {
        const float *pt = a.partial + size_t(tile) * slices * n * 64 + lane;
        for (int m0 = 0; m0 < c; m0 += MT) {
          float acc[MT];
          dev::sum_slices<MT, 4>(
              acc, [&](int s, int m) { return pt + (size_t(s) * n + pl.pos[min(m0 + m, c - 1)]) * 64; }, slices);
#pragma unroll
          for (int m = 0; m < MT; ++m)
            if (m0 + m < c) finish(pl.pos[m0 + m], acc[m]);
        }
        dev::reset_counter(ctr, lane);
      }
    }
    if (!DOWN) return;
    if (last) last = dev::last_arrival(&a.counters[(size_t(tiles) * slots + tile) * kCounterStride],
                                       unsigned(pl.active), lane);
    if (lane == 0) owner = last;
  }
  if (!DOWN) return;
  __syncthreads();
  if (!owner) return;

  // expert combine: lane (r, j) of wave w sums row r for tokens w*L + j,
  // (w+4)*L + j, ...  The y values and probabilities of CT tokens x CR routes
  // load in one branch-free batch (indices clamped in range, out-of-range
  // entries dropped when summing), then add up in route order.
  if (row < nout) {
    constexpr int CT = 4, CR = 8;
    const int T = 4 * L;
    for (int t0 = wave * L + j; t0 < a.rows; t0 += CT * T) {
      float acc[CT];
#pragma unroll
      for (int q = 0; q < CT; ++q) acc[q] = 0.0f;
      for (int r0 = 0; r0 < a.topk; r0 += CR) {
        int R[CT][CR];
        float v[CT][CR], pv[CT][CR];
#pragma unroll
        for (int q = 0; q < CT; ++q)
#pragma unroll
          for (int u = 0; u < CR; ++u) {
            const int tk = min(t0 + q * T, a.rows - 1), r = min(r0 + u, a.topk - 1);
            R[q][u] = tk * a.topk + pl.ord[tk * a.topk + r];
          }
#pragma unroll
        for (int q = 0; q < CT; ++q)
#pragma unroll
          for (int u = 0; u < CR; ++u) {
            pv[q][u] = a.routes[n + R[q][u]];
            v[q][u] = dev::xload(a.y + size_t(R[q][u]) * a.hidden + row);
          }
#pragma unroll
        for (int q = 0; q < CT; ++q)
#pragma unroll
          for (int u = 0; u < CR; ++u) {
            const bool ok = t0 + q * T < a.rows && r0 + u < a.topk && pl.ids[R[q][u]] < uint32_t(a.experts);
            if (ok) acc[q] = add_mul_nofma(acc[q], v[q][u], pv[q][u]);  // moe.comp:70 / :126: out + y*p
          }
      }
#pragma unroll
      for (int q = 0; q < CT; ++q)
        if (t0 + q * T < a.rows) a.out[size_t(t0 + q * T) * a.hidden + row] = acc[q];
    }
  }
  if (wave == 0) dev::reset_counter(&a.counters[(size_t(tiles) * slots + tile) * kCounterStride], lane);
}

template <int MT, int GSW>
void launch_mt(const MoELaunch &a, const MoEPlanSizes &p, hipStream_t s) {
  const int tgu = 2 * a.gu.blocks, tdn = a.dn.blocks;
  const int ggu = (tgu + 7) / 8 * 8 * p.slots * p.slices_gu;
  const int gdn = (tdn + 7) / 8 * 8 * p.slots * p.slices_dn;
  hipLaunchKernelGGL(k_moe_plan, dim3(p.slots + 1), dim3(64), 0, s, a, p.slots);
  hipLaunchKernelGGL((k_moe<MT, GSW, false>), dim3(ggu), dim3(256), p.lds_gu, s, a, p.slices_gu, p.sps_gu, p.slots);
  hipLaunchKernelGGL((k_moe<MT, GSW, true>), dim3(gdn), dim3(256), p.lds_dn, s, a, p.slices_dn, p.sps_dn, p.slots);
}

// ---- one token, one launch -----------------------------------------------
// With one token the k routed experts form a block-structured MLP: gate/up of
// every expert reads the same x, and the down projections add up as
//     out = sum_j p_j W_d[e_j] h_j  (j in ascending expert id),
// i.e. a down matvec over the concatenated h whose K-segments use expert
// e_j's weights.  So the layer runs as the fused decode MLP runs (qnn_mlp.hip):
// workgroup w takes gate/up item w and down item w; the down weights go to
// LDS together with the gate/up weights; a down item waits only for the
// blocks of h its K-slice reads (per-(slot, block) epoch flags); and the
// split-K combine of a down block, done by the last of its k * slices
// arrivals, sums each expert's slices in order and then the experts in
// ascending id with p, which is exactly the arithmetic of the two-launch path
// (k_moe), so the results are bit-identical to it.
//
// Items: gate/up tiles are whole waves over one matrix (gate or up) of one
// (slot, 64-row block) pair, numbered 2*pair + up over all slots and mapped
// like the dense SwiGLU (units padded to 16: the gate tile u and the up tile
// u + 8 share an XCD).  Down units are (slot, block) with blocks padded to 8
// per slot, so every arrival of a down block has the same blockIdx % 8.
size_t moe_decode_lds(int g) { return dev::xplanes_bytes(1, 4 * g); }

// Phase timestamps of k_moe_decode, built only into libqnn_hip_trace.so
// (-DQNN_PHASE_TRACE), as in the fused decode MLP: thread 0 of workgroup wg
// stores the device's real-time counter (100 MHz) at phase k; nothing else
// changes.
#ifdef QNN_PHASE_TRACE
constexpr int kMoEPhaseWGs = 2048, kMoEPhases = 16;
__device__ unsigned long long g_moe_phase[kMoEPhaseWGs * kMoEPhases];
#define QNN_MOE_PHASE(k)                                                                             \
  do {                                                                                               \
    if (threadIdx.x == 0 && blockIdx.x < kMoEPhaseWGs)                                               \
      g_moe_phase[blockIdx.x * kMoEPhases + (k)] = __builtin_amdgcn_s_memrealtime();                 \
  } while (0)
#else
#define QNN_MOE_PHASE(k) \
  do {                   \
  } while (0)
#endif

// J > 0: the token's routes are computed here from a.logits (GO_MOE_ROUTE
// recorded just before, J = experts/64 rounded up to a power of two), by every
// wave with the route op's own code, and workgroup 0 writes them to the
// route tensor as the route op would.
template <int GG, int GD, int J>
__global__ __launch_bounds__(256) void k_moe_decode(const MoELaunch a, const int sps_gu, const int slices_gu,
                                                    const int sps_dn, const int slices_dn, const int units_gu,
                                                    const int bpad_dn, const int grid_dn) {
  extern __shared__ uint4 dyn_lds[];
  __shared__ float red[4][64];
  const int wave = dev::wave_id(), tid = threadIdx.x, lane = tid & 63, part = wave;
  const int wg = blockIdx.x;
  const int k = a.topk;
  constexpr int QD = dev::scale_quads<GD>();
  constexpr int XG = 4 * (GG > GD ? GG : GD);
  const dev::XPlanes xs = dev::xplanes_at(dyn_lds, 1, XG);
  const I4Layout &lg = a.gu, &ld = a.dn;
  QNN_MOE_PHASE(0);

  // ---- route ranks: lane i < k holds route i; rank = its position in
  //      ascending expert id (ties: lower route index, reported as invalid).
  uint32_t id;
  float prob = 0.0f;  // J > 0: computed once the weight loads are issued
  dev::RouteRow<(J > 0 ? J : 1)> rr_;
  if constexpr (J == 0) {
    const dev::Rsrc rr = dev::rsrc(a.routes, size_t(2 * k) * 4);  // branch-free loads (past the end: 0)
    const uint32_t id0 = __float_as_uint(dev::ld32f(rr, uint32_t(lane) * 4u, 0));
    const float prob0 = dev::ld32f(rr, uint32_t(k + lane) * 4u, 0);
    id = lane < k ? id0 : 0xFFFFFFFFu;
    prob = lane < k ? prob0 : 0.0f;
  } else {
    __shared__ unsigned long long rsel[4][64];
    __shared__ int rids[4][64];
    __shared__ float rlv[4][64];
    dev::route_select<J>(rr_, a.logits, a.experts, k, lane, rsel[wave], rids[wave], rlv[wave]);
    id = lane < k ? uint32_t(rr_.id) : 0xFFFFFFFFu;
  }
  int rank = 0;
  bool dup = false;
  for (int i = 0; i < k; ++i) {
    const uint32_t o = uint32_t(__builtin_amdgcn_readlane(int(id), i));
    rank += (o < id) || (o == id && i < lane);
    dup |= o == id && i != lane;
  }
  if (wg == 0 && wave == 0 && __ballot(lane < k && (dup || id >= uint32_t(a.experts))) != 0 && lane == 0)
    atomicOr(a.err, 8);
  auto src_of = [&](int slot) { return __ffsll((unsigned long long)__ballot(lane < k && rank == slot)) - 1; };
  auto expert_of = [&](int slot) {  // clamped so addresses stay inside the set; scalar (uniform) for the resources
    return __builtin_amdgcn_readfirstlane(
        int(min(uint32_t(__builtin_amdgcn_readlane(int(id), src_of(slot))), uint32_t(a.experts - 1))));
  };

  // ---- gate/up item
  const int pairs = k * lg.blocks;
  int unit = 0, slice = 0;
  const bool mapped = dev::map_tile(wg, slices_gu, units_gu, unit, slice);
  const int tile_m = 2 * ((unit >> 4) * 8 + (unit & 7)) + ((unit >> 3) & 1);
  const bool gu_on = mapped && tile_m < 2 * pairs;
  const int tile = gu_on ? tile_m : 0;
  if (!gu_on) slice = 0;
  const int pair = tile >> 1, slot = pair / lg.blocks, blk = pair - slot * lg.blocks;
  const int ws0 = slice * 4 * sps_gu, s0 = ws0 + part * sps_gu;
  const int ns = max(0, min(sps_gu, lg.steps - s0));
  const int sgroups = min(4 * sps_gu, lg.groups - ws0);

  // ---- down item
  int ud = 0, sld = 0;
  bool dn_on = wg < grid_dn && dev::map_tile(wg, slices_dn, k * bpad_dn, ud, sld);
  int dslot = ud / bpad_dn, td = ud - dslot * bpad_dn;
  dn_on = dn_on && td < ld.blocks;
  if (!dn_on) dslot = td = sld = 0;
  const int wsd = sld * 4 * sps_dn, s0d = wsd + part * sps_dn;
  const int nsd = max(0, min(sps_dn, ld.steps - s0d));
  const int sgd = min(4 * sps_dn, ld.groups - wsd);

  const int eg = expert_of(slot);

  // ---- 1) loads: x slice and gate/up weights to registers
  float4 xr[1][dev::x_iters<GG>()];
  uint4 w[GG];
  uint4 q[dev::scale_quads<GG>()];
  dev::load_x<1, GG>(xr, dev::rsrc(a.x, size_t(a.hidden) * 4), [](int) { return 0u; }, 1, ws0 * 32, sgroups * 32,
                     tid);
  {
    const uint8_t *wb = a.gate_up + size_t(2 * eg + (tile & 1)) * a.gu_stride;
    dev::load_wq<GG>(w, q, dev::block_nib_rsrc(wb, lg, blk), dev::block_scl_rsrc(wb + lg.nib_bytes(), lg, blk), lg,
                     blk, s0, lane);
  }
  float sc[GG];
  dev::pick_scales<GG>(sc, q, s0);
  if constexpr (J > 0) {  // the probabilities, while the loads are in flight
    prob = dev::route_probs<J>(rr_, a.experts, k, a.normalize, lane);
    if (wg == 0 && wave == 0 && lane < k) {
      a.routes_out[lane] = __uint_as_float(uint32_t(rr_.id));
      a.routes_out[k + lane] = prob;
    }
  }

  // ---- 2) gate/up: dot, parts in LDS, split-K exchange; the last of the
  //         2 x slices arrivals of a pair writes its h rows and raises its flag.
  dev::stage_x<1, GG>(xs, xr, 1, ws0 * 32, sgroups * 32, a.hidden, tid, lane);
  __syncthreads();
  QNN_MOE_PHASE(1);
  float acc[1] = {0.0f};
  if (ns > 0) {
    dev::XPlanes xp = xs;
    const int g0 = part * sps_gu;
    xp.q = xs.q + size_t(g0) * dev::kXWords;
    xp.s2 = xs.s2 + g0;
    xp.off = xs.off + g0;
    dev::dot<1, GG>(acc, w, sc, xp, 1, 0, ns);
  }
  if (part > 0) red[part][lane] = acc[0];
  __syncthreads();
  QNN_MOE_PHASE(2);
  if (part == 0 && gu_on) {
    acc[0] = ((acc[0] + red[1][lane]) + red[2][lane]) + red[3][lane];
    dev::xstore(a.partial + (size_t(tile) * slices_gu + slice) * 64 + lane, acc[0]);
    unsigned *ctr = &a.counters[size_t(pair) * kCounterStride];
    if (dev::last_arrival(ctr, unsigned(2 * slices_gu), lane)) {
      const float *pt = a.partial + size_t(tile & ~1) * slices_gu * 64 + lane;
      float gu[2];  // gate and up, their slices loaded in one batch
      dev::sum_slices<2, 16>(gu, [&](int s, int m) { return pt + size_t(m * slices_gu + s) * 64; }, slices_gu);
      QNN_MOE_PHASE(11);
      dev::reset_counter(ctr, lane);
      const int row = blk * 64 + lane;
      if (row < a.inter) dev::xstore(a.h + size_t(slot) * a.inter + row, dev::silu(gu[0]) * gu[1]);
      __builtin_amdgcn_s_waitcnt(0);  // the block's h is at the coherence point
      if (lane == 0)
        __hip_atomic_store(a.flags + size_t(pair) * 64, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      QNN_MOE_PHASE(4);
    }
    QNN_MOE_PHASE(3);
  }
  if (!dn_on) return;

  // ---- down weights to registers, issued only now, so that the gate/up
  //      weights of every workgroup are requested first and h is complete
  //      sooner.
  uint4 wd[GD];
  uint4 qd[QD];
  {
    const int ed = expert_of(dslot);  // after the gate/up loads are issued
    const uint8_t *db = a.down + size_t(ed) * a.dn_stride;
    dev::load_wq<GD>(wd, qd, dev::block_nib_rsrc(db, ld, td), dev::block_scl_rsrc(db + ld.nib_bytes(), ld, td), ld,
                     td, s0d, lane);
  }
  // Lane j: the probability of slot j (ascending expert id), for the down
  // combine, taken now rather than on the combine's dependent path.
  float pslot = 0.0f;
  for (int j = 0; j < k; ++j) {
    const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prob), src_of(j)));
    if (lane == j) pslot = pj;
  }

  // ---- 3) down: wait for the blocks of h_slot in the K-slice, stage, dot
  //         with the weights in registers, split-K exchange; the last arrival
  //         of the block combines slices and experts.
  __syncthreads();  // xs and red are reused
  if (wave == 0) {
    const int b0 = (wsd * 32) >> 6, nb = (sgd * 32 + 63) >> 6;  // h blocks of the slice (<= 64)
    const unsigned *fl = a.flags + (size_t(dslot) * lg.blocks + b0) * 64;
    unsigned spins = 0;
    for (;;) {
      const bool ready =
          lane >= nb || __hip_atomic_load(fl + size_t(lane) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
      if (__ballot(!ready) == 0) break;
      __builtin_amdgcn_s_sleep(1);
      if (++spins > (1u << 25)) {  // ~1 s: report and finish instead of hanging
        if (lane == 0) atomicOr(a.err, 2);
        break;
      }
    }
  }
  __syncthreads();
  QNN_MOE_PHASE(5);
  float4 hr[1][dev::x_iters<GD>()];
  dev::load_x<1, GD, dev::kCoherent>(hr, dev::rsrc(a.h + size_t(dslot) * a.inter, size_t(a.inter) * 4),
                                    [](int) { return 0u; }, 1, wsd * 32, sgd * 32, tid);
  dev::stage_x<1, GD>(xs, hr, 1, wsd * 32, sgd * 32, a.inter, tid, lane);
  __syncthreads();
  QNN_MOE_PHASE(6);
  float scd[GD];
  dev::pick_scales<GD>(scd, qd, s0d);
  acc[0] = 0.0f;
  if (nsd > 0) {
    dev::XPlanes xp = xs;
    const int g0 = part * sps_dn;
    xp.q = xs.q + size_t(g0) * dev::kXWords;
    xp.s2 = xs.s2 + g0;
    xp.off = xs.off + g0;
    dev::dot<1, GD>(acc, wd, scd, xp, 1, 0, nsd);
  }
  if (part > 0) red[part][lane] = acc[0];
  __syncthreads();
  QNN_MOE_PHASE(7);
  if (part > 0) return;
  acc[0] = ((acc[0] + red[1][lane]) + red[2][lane]) + red[3][lane];
  dev::xstore(a.partial_dn + ((size_t(td) * k + dslot) * slices_dn + sld) * 64 + lane, acc[0]);
  unsigned *ctr = &a.counters_dn[size_t(td) * kCounterStride];
  const bool last = dev::last_arrival(ctr, unsigned(k * slices_dn), lane);
  QNN_MOE_PHASE(9);
  if (!last) return;
  const float *pt = a.partial_dn + size_t(td) * k * slices_dn * 64 + lane;
  // The k x slices partial sums (expert-major) load 32 at a time; each
  // expert's y sums its slices in slice order, and out adds the experts in
  // ascending id order.
  float out = 0.0f, y = 0.0f;
  const int total = k * slices_dn;
  for (int i0 = 0; i0 < total; i0 += 16) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i0 + i < total) v[i] = dev::xload(pt + size_t(i0 + i) * 64);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i0 + i < total) {
        const int j = (i0 + i) / slices_dn, s = i0 + i - j * slices_dn;
        y = s == 0 ? v[i] : y + v[i];
        if (s == slices_dn - 1)  // moe.comp:70 / :126: out + y*p
          out = add_mul_nofma(out, y, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pslot), j)));
      }
  }
  QNN_MOE_PHASE(10);
  dev::reset_counter(ctr, lane);
  const int row = td * 64 + lane;
  if (row < a.hidden) a.out[row] = out;
  QNN_MOE_PHASE(8);
}

template <int G, int J>
bool decode_launch(const MoELaunch &a, const MoEPlanSizes &p, const MoEDecodePlan &d, hipStream_t s) {
  hipLaunchKernelGGL((k_moe_decode<G, G, J>), dim3(d.grid), dim3(256), moe_decode_lds(G), s, a, p.sps_gu,
                     p.slices_gu, p.sps_dn, p.slices_dn, d.units_gu, d.bpad_dn, d.grid_dn);
  return hipGetLastError() == hipSuccess;
}

template <int G, int J>
int decode_capacity(int device) {
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(&k_moe_decode<G, G, J>),
                                                   256, moe_decode_lds(G)) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return per_cu * cus;
}

}  // namespace

MoEPlanSizes moe_plan(const MoELaunch &a) {
  if (a.gu.lanes != 1 || a.dn.lanes != 1) fail(QNN_E_INVALID_OP, "MoE expert layouts need one lane per row");
  MoEPlanSizes p;
  const int n = a.rows * a.topk;
  p.slots = std::min(a.experts, n);
  // One token per pass: fewer registers (at 4 steps per wave 97-114 VGPRs
  // against 123-126 at 2 tokens); measured faster at 4, 16 and 32 tokens (16:
  // 159 against 167 us, 100.7 against 123.2 us with the current kernels) even
  // though an expert with several tokens makes several passes over its
  // weights in registers.  QNN_MOE_MT (1, 2, 4) overrides.
  p.mt = 1;
  const int fmt = tuning().moe_mt;
  if (fmt == 1 || fmt == 2 || fmt == 4) p.mt = fmt;
  // Steps per wave: 8 with one token per pass, 4 with several, measured
  // fastest for 128 experts of 768 x 2048 (one token per pass, 2-64 rows: 8
  // steps 4-17% faster than 4, e.g. 16 rows 129 -> 114 us, 100.7 against
  // 118.3 us with the current kernels; 2 tokens per pass: 4 steps 14-16%
  // faster than 2 and than 8).  One row with its routes given would take 4
  // (13.36 against 13.63 us), but the launch that computes the routes itself
  // is faster at 8 (16.55 against 17.91 us) and must sum in the same order as
  // the routes-given launch, so one row keeps 8.  QNN_MOE_SPS overrides.
  // Bounded by the activation-slice LDS budget.
  const int forced = tuning().moe_sps;
  auto steps = [&](const I4Layout &l, int) {
    const int lds_cap = int((48 << 10) / (size_t(p.mt) * 4 * l.lanes * (dev::kXWords * 4 + 8)));
    const int cap = std::max(1, std::min(8, lds_cap));
    return std::min(forced > 0 ? forced : (p.mt == 1 ? 8 : 4), cap);
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
  p.plan_words = size_t(p.slots) * kSlotWords + 2 * size_t(n);
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

MoEDecodePlan moe_decode_plan(const MoELaunch &a, const MoEPlanSizes &p) {
  MoEDecodePlan d;
  if (a.rows != 1 || p.mt != 1 || a.gu.lanes != 1 || a.dn.lanes != 1 || p.sps_gu != p.sps_dn) return d;
  if (p.gsw != 1 && p.gsw != 2 && p.gsw != 4 && p.gsw != 8) return d;
  const int k = a.topk;
  const int pairs = k * a.gu.blocks;
  d.units_gu = (2 * pairs + 15) / 16 * 16;
  d.bpad_dn = (a.dn.blocks + 7) / 8 * 8;
  d.grid_dn = k * d.bpad_dn * p.slices_dn;
  d.grid = std::max(d.units_gu * p.slices_gu, d.grid_dn);
  d.partial_gu = size_t(2 * pairs) * p.slices_gu * 64;
  d.partial_dn = size_t(a.dn.blocks) * k * p.slices_dn * 64;
  d.counters_gu = size_t(pairs) * kCounterStride;
  d.counters_dn = size_t(a.dn.blocks) * kCounterStride;
  d.flag_bytes = size_t(pairs) * 256;
  d.ok = true;
  return d;
}

// Route-computing variants exist for the default one-token plan (8 steps per
// wave); a forced plan uses the route op and the plain variant.
int moe_route_j(int experts) {
  const int j = (experts + 63) / 64;
  return j <= 1 ? 1 : (j <= 2 ? 2 : (j <= 4 ? 4 : (j <= 8 ? 8 : (j <= 16 ? 16 : 0))));
}

int moe_phase_read(void *dst, size_t bytes) {
#ifdef QNN_PHASE_TRACE
  const size_t n = std::min(bytes, sizeof(g_moe_phase));
  if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_moe_phase), n, 0, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  static const unsigned long long zeros[kMoEPhaseWGs * kMoEPhases] = {};
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_moe_phase), zeros, sizeof(g_moe_phase), 0, hipMemcpyHostToDevice) != hipSuccess)
    return -1;
  return int(n / 8);
#else
  (void)dst;
  (void)bytes;
  return -2;
#endif
}

int moe_decode_capacity(const MoEPlanSizes &p, int route_j, int device) {
  if (route_j) {
    if (p.gsw != 8) return 0;
    switch (route_j) {
      case 1: return decode_capacity<8, 1>(device);
      case 2: return decode_capacity<8, 2>(device);
      case 4: return decode_capacity<8, 4>(device);
      case 8: return decode_capacity<8, 8>(device);
      case 16: return decode_capacity<8, 16>(device);
      default: return 0;
    }
  }
  switch (p.gsw) {
    case 1: return decode_capacity<1, 0>(device);
    case 2: return decode_capacity<2, 0>(device);
    case 4: return decode_capacity<4, 0>(device);
    case 8: return decode_capacity<8, 0>(device);
    default: return 0;
  }
}

bool moe_decode_launch(const MoELaunch &a, const MoEPlanSizes &p, const MoEDecodePlan &d, int route_j, hipStream_t s) {
  if (route_j) {
    if (p.gsw != 8) return false;
    switch (route_j) {
      case 1: return decode_launch<8, 1>(a, p, d, s);
      case 2: return decode_launch<8, 2>(a, p, d, s);
      case 4: return decode_launch<8, 4>(a, p, d, s);
      case 8: return decode_launch<8, 8>(a, p, d, s);
      case 16: return decode_launch<8, 16>(a, p, d, s);
      default: return false;
    }
  }
  switch (p.gsw) {
    case 1: return decode_launch<1, 0>(a, p, d, s);
    case 2: return decode_launch<2, 0>(a, p, d, s);
    case 4: return decode_launch<4, 0>(a, p, d, s);
    case 8: return decode_launch<8, 0>(a, p, d, s);
    default: return false;
  }
}

}  // namespace qnn
