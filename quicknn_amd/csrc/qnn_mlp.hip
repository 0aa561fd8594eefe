// qnn_mlp.hip -- persistent decode kernel for a stack of native-INT4 MLP layers.
//
// One cooperative launch runs L layers of
//     h_l = silu(G_l x_l) * (U_l x_l);   x_{l+1} = D_l h_l
// (the per-layer sequence TrySwiGLUVector + Int4Linear of the decode loop,
// src/models/QuickNN.Models.QwenHybrid.pas:692-702), with x_L written to the
// output.  Separate launches cost a kernel boundary each (a few microseconds,
// as much as a whole 16 MB matvec at HBM speed); here the boundaries are
// replaced by per-tile readiness flags:
//
//  * Work is split into items exactly as in the per-op kernel (qnn_int4.hip):
//    a 256-thread workgroup owns a 64-row tile (gate/up: 32 gate + 32 up rows)
//    and a K-slice of 4*GSW groups.  Workgroup j always takes items j, j+P, ...
//    of every phase, in phase order.
//  * Before waiting for its inputs a workgroup issues the weight loads of its
//    item: weights do not depend on activations, so HBM streaming overlaps the
//    dependency wait.
//  * The last slice of a tile to finish (atomic ticket) sums the slices in
//    order, writes the tile's outputs and raises the tile's flag to
//    epoch*2^16 + layer + 1.  Consumers poll only the flags of the tiles that
//    produce their K-slice.  The epoch is a device counter advanced by the
//    last workgroup to exit, so flags, tickets and the exit counter are
//    self-resetting (no memsets between launches).
//  * Every cross-workgroup value travels as a device-scope atomic store/load
//    (coherent across XCDs); writers wait for completion before raising a
//    flag or taking a ticket.
//  * Co-residency of all workgroups is guaranteed by the cooperative launch;
//    every spin is bounded: on timeout the kernel records an error and all
//    waits give up, so every wave always exits.
//
// Deadlock freedom: a workgroup processes its items in phase order, and every
// item of phase p depends only on phase p-1.  The earliest incomplete phase
// therefore always has all of its inputs and its holders are not blocked.
#include "qnn_internal.h"

namespace qnn {
namespace {

__device__ __forceinline__ float silu_dev(float g) {
  return g >= 20.0f ? g : (g <= -20.0f ? 0.0f : g / (1.0f + expf(-g)));
}
__device__ __forceinline__ uint32_t sel4u(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ float ld_coh(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void mem_complete() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

constexpr int kFlagStride = 8;  // uint64 flags 64 bytes apart

// Thread 0 polls flags [first, last] until all reach `target`; the workgroup
// then proceeds.  Bounded: after `limit` polls the error word is set, the
// abort word is raised and every later wait returns at once.
__device__ void wait_tiles(const MlpArgs &a, const unsigned long long *flags, int first, int last,
                           unsigned long long target) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    for (int t = first; t <= last; ++t) {
      while (__hip_atomic_load(&flags[size_t(t) * kFlagStride], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
             target) {
        if (__hip_atomic_load(a.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        if (++spins > a.spin_limit) {
          atomicOr(a.err, 2);
          __hip_atomic_store(a.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
  }
  __syncthreads();
}

// One work item: 64 rows x (4*GSW groups).  SWIGLU: wave tile `tile` covers
// output rows 32*tile..+31, gate rows in lanes 0-31 and up rows in 32-63.
template <int GSW, bool SWIGLU>
__device__ void mlp_item(const MlpArgs &a, const int layer, const int tile, const int slice, const int slices,
                         const int g4, const int kdim, const int nout, const uint4 *nibA, const float *sclA,
                         const uint4 *nibB, const float *sclB, const float *xsrc, const unsigned long long *in_flags,
                         const int in_rows_per_tile, const unsigned long long in_target, float *part, unsigned *tick,
                         float *out, unsigned long long *out_flags, const unsigned long long out_value) {
  constexpr int GS = 4 * GSW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g0 = slice * GS;
  const int ng = min(GS, g4 - g0);
  const int gw0 = wave * GSW;
  const int ngw = max(0, min(GSW, ng - gw0));

  // 1) Weights of this item (independent of activations).
  int stile = tile, srow = lane;
  const uint4 *nb = nibA;
  const float *sb = sclA;
  if (SWIGLU) {
    stile = tile >> 1;
    srow = (tile & 1) * 32 + (lane & 31);
    if (lane >= 32) { nb = nibB; sb = sclB; }
  }
  const int gq0 = g0 + gw0;
  const uint4 *nib = nb + (size_t(stile) * g4 + gq0) * 64 + srow;
  const float *sclf = sb + (size_t(stile) * (g4 >> 2) + (gq0 >> 2)) * 256 + srow * 4;
  uint4 w[GSW];
  float sc[GSW];
#pragma unroll
  for (int g = 0; g < GSW; ++g)
    if (g < ngw) {
      const int gg = gq0 + g;
      sc[g] = sclf[((gg >> 2) - (gq0 >> 2)) * 256 + (gg & 3)];
    }
#pragma unroll
  for (int g = 0; g < GSW; ++g)
    if (g < ngw) w[g] = nib[g * 64];

  // 2) Wait for the producer tiles of this K-slice.
  const int k0 = g0 * 32, k1 = min(kdim, (g0 + ng) * 32);
  if (in_flags && k1 > k0) wait_tiles(a, in_flags, k0 / in_rows_per_tile, (k1 - 1) / in_rows_per_tile, in_target);

  // 3) x slice (coherent loads: written by other workgroups) + group sums.
  __shared__ float xs[GS * 32];
  __shared__ float xsum[GS];
  __shared__ float red[3][64];
  constexpr int XIT = (GS * 32 + 1023) / 1024;
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int e = (it * 256 + tid) * 4;
    const int kk = k0 + e;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e < ng * 32) {
      if (kk < kdim) v.x = ld_coh(xsrc + kk);
      if (kk + 1 < kdim) v.y = ld_coh(xsrc + kk + 1);
      if (kk + 2 < kdim) v.z = ld_coh(xsrc + kk + 2);
      if (kk + 3 < kdim) v.w = ld_coh(xsrc + kk + 3);
    }
    if (e < GS * 32) *reinterpret_cast<float4 *>(&xs[e]) = v;
    float p = (v.x + v.y) + (v.z + v.w);
    p += __shfl_xor(p, 1);
    p += __shfl_xor(p, 2);
    p += __shfl_xor(p, 4);
    if ((lane & 7) == 0 && e < GS * 32) xsum[e >> 5] = p;
  }
  __syncthreads();

  // 4) Dequantise and accumulate this wave's groups.
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < GSW; ++g) {
    if (g < ngw) {
      const int gl = gw0 + g;
      const float4 *xv = reinterpret_cast<const float4 *>(&xs[gl * 32]);
      float pc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t wd = sel4u(w[g], c);
        const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
        const float4 xa = xv[2 * c], xb = xv[2 * c + 1];
        float t = float(lo & 0xFFu) * xa.x;
        t = fmaf(float(hi & 0xFFu), xa.y, t);
        t = fmaf(float((lo >> 8) & 0xFFu), xa.z, t);
        t = fmaf(float((hi >> 8) & 0xFFu), xa.w, t);
        t = fmaf(float((lo >> 16) & 0xFFu), xb.x, t);
        t = fmaf(float((hi >> 16) & 0xFFu), xb.y, t);
        t = fmaf(float(lo >> 24), xb.z, t);
        t = fmaf(float(hi >> 24), xb.w, t);
        pc[c] = t;
      }
      const float pg = (pc[0] + pc[1]) + (pc[2] + pc[3]);
      acc = fmaf(sc[g], pg - 8.0f * xsum[gl], acc);
    }
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    acc = ((acc + red[0][lane]) + red[1][lane]) + red[2][lane];
    bool last = true;
    if (slices > 1) {
      st_coh(part + (size_t(tile) * slices + slice) * 64 + lane, acc);
      mem_complete();
      unsigned ticket = 0;
      if (lane == 0)
        ticket = __hip_atomic_fetch_add(&tick[tile * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ticket = __shfl(ticket, 0);
      last = ticket == unsigned(slices - 1);
      if (last) {
        const float *pt = part + size_t(tile) * slices * 64 + lane;
        acc = 0.0f;
        for (int s0 = 0; s0 < slices; s0 += 16) {
          float v[16];
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (s0 + j < slices) v[j] = ld_coh(pt + size_t(s0 + j) * 64);
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (s0 + j < slices) acc += v[j];
        }
        if (lane == 0)
          __hip_atomic_store(&tick[tile * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (last) {
      if (SWIGLU) {
        const float u = __shfl_down(acc, 32);
        const int row = tile * 32 + lane;
        if (lane < 32 && row < nout) st_coh(out + row, silu_dev(acc) * u);
      } else {
        const int row = tile * 64 + lane;
        if (row < nout) st_coh(out + row, acc);
      }
      mem_complete();
      if (lane == 0)
        __hip_atomic_store(&out_flags[size_t(tile) * kFlagStride], out_value, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();  // xs/red are reused by the next item
}

template <int GSWU, int GSWD>
__global__ __launch_bounds__(256) void k_int4_mlp_stack(const MlpArgs a) {
  __shared__ unsigned long long epoch_sh;
  if (threadIdx.x == 0)
    epoch_sh = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
  __syncthreads();
  const unsigned long long base = epoch_sh << 16;
  const int P = gridDim.x;
  const int n_gu = a.tiles_gu * a.slices_gu, n_d = a.tiles_d * a.slices_d;
  for (int l = 0; l < a.layers; ++l) {
    const MlpLayerPtrs lw = a.w[l];
    const float *x = l == 0 ? a.x0 : a.ybuf + size_t((l - 1) & 1) * a.hidden;
    float *h = a.hbuf + size_t(l & 1) * a.inter;
    float *y = l == a.layers - 1 ? a.out : a.ybuf + size_t(l & 1) * a.hidden;
    // Phase GU(l): needs x_l (D tiles of layer l-1: flag >= base + l).
    for (int it = blockIdx.x; it < n_gu; it += P) {
      const int q = it / a.slices_gu;
      const int tile = q, slice = it - q * a.slices_gu;
      mlp_item<GSWU, true>(a, l, tile, slice, a.slices_gu, a.g4_gu, a.hidden, a.inter, lw.gnib, lw.gscl, lw.unib,
                           lw.uscl, x, l == 0 ? nullptr : a.flag_d, 64, base + l, a.part_gu, a.tick_gu, h, a.flag_gu,
                           base + l + 1);
    }
    // Phase D(l): needs h_l (GU tiles of layer l: flag >= base + l + 1).
    for (int it = blockIdx.x; it < n_d; it += P) {
      const int q = it / a.slices_d;
      const int tile = q, slice = it - q * a.slices_d;
      mlp_item<GSWD, false>(a, l, tile, slice, a.slices_d, a.g4_d, a.inter, a.hidden, lw.dnib, lw.dscl, nullptr,
                            nullptr, h, a.flag_gu, 32, base + l + 1, a.part_d, a.tick_d, y, a.flag_d, base + l + 1);
    }
  }
  // Exit ticket: the last workgroup advances the epoch (all others have read it).
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = __hip_atomic_fetch_add(a.exit_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == unsigned(P - 1)) {
      __hip_atomic_store(a.exit_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.abort, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.epoch, epoch_sh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

const void *mlp_kernel(int gswu, int gswd) {
  if (gswu == 20 && gswd == 16) return reinterpret_cast<const void *>(&k_int4_mlp_stack<20, 16>);
  if (gswu == 20) return reinterpret_cast<const void *>(&k_int4_mlp_stack<20, 8>);
  if (gswd == 16) return reinterpret_cast<const void *>(&k_int4_mlp_stack<8, 16>);
  return gswu == 4 ? reinterpret_cast<const void *>(&k_int4_mlp_stack<4, 8>)
                   : reinterpret_cast<const void *>(&k_int4_mlp_stack<8, 8>);
}

int mlp_stack_grid(int gswu, int gswd, int want) {
  int per_cu = 0, dev = 0, cus = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
  hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, mlp_kernel(gswu, gswd), 256, 0), "occupancy");
  if (per_cu < 1) fail(QNN_E_NOT_SUPPORTED, "MLP stack kernel cannot be resident");
  return std::max(1, std::min(want, per_cu * cus));
}

void mlp_stack_launch(const MlpArgs &a, int gswu, int gswd, int grid, hipStream_t st) {
  void *args[] = {const_cast<MlpArgs *>(&a)};
  hip_check(hipLaunchCooperativeKernel(mlp_kernel(gswu, gswd), dim3(grid), dim3(256), args, 0, st),
            "cooperative MLP launch");
}

}  // namespace qnn
