// qnn_exchange.h -- split-K exchange between the workgroups of one tile, and
// the tile map (shared by the INT4, MoE, fused-MLP and GGUF kernels).
//
// A K-split tile's workgroups each store a partial sum and take a ticket; the
// last arrival sums the partials in slice order, so results do not depend on
// timing.  Partials travel as device-scope (write-through) stores and loads,
// which are coherent across XCDs by themselves, so the exchange is correct
// wherever the device places the workgroups (a device-scope fence would
// write back and invalidate the whole L2 instead).  Reading them through one
// XCD's L2 when every slice ran there was measured too: it only made the
// rarely run, instruction-cache-cold combine code larger and the kernels
// slower.
#pragma once
#include "qnn_internal.h"
#include "qnn_lanes.h"

namespace qnn {
namespace dev {

// LDS ordering between the lanes of one wave (LDS operations of a wave run in
// order; this keeps the compiler from moving them across).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void xstore(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float xload(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  ticket = __builtin_amdgcn_readfirstlane(ticket);  // lane 0's (every lane is active)
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
__device__ __forceinline__ void sum_slices(float (&acc)[MT], AddrF part, int slices) {
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
  for (int s0 = 0; s0 < slices; s0 += PU) {
    float v[PU][MT];
#pragma unroll
    for (int j = 0; j < PU; ++j)
      if (s0 + j < slices)
#pragma unroll
        for (int m = 0; m < MT; ++m) v[j][m] = xload(part(s0 + j, m));
#pragma unroll
    for (int j = 0; j < PU; ++j)
      if (s0 + j < slices)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] += v[j][m];
  }
}

// blockIdx -> (unit, rest): the workgroups of a unit have the same
// blockIdx % 8 and consecutive blockIdx / 8, so they are dispatched together
// (and, with the device's usual round-robin dealing, on one XCD).  `per` =
// workgroups per unit.
__device__ __forceinline__ bool map_tile(int b, int per, int units, int &unit, int &rest) {
  const int xcd = b & 7, k = b >> 3;
  const int q = k / per;
  unit = q * 8 + xcd;
  rest = k - q * per;
  return unit < units;
}

}  // namespace dev
}  // namespace qnn
