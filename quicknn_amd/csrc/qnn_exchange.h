// qnn_exchange.h -- split-K exchange between the workgroups of one tile, and
// the XCD-aware tile map (shared by the INT4, MoE, fused-MLP and GGUF kernels).
//
// A K-split tile's workgroups each store a partial sum and take a ticket; the
// last arrival sums the partials in slice order.  Partials are always stored
// write-through at device scope, so they are at the coherence point whichever
// XCD wrote them.  The last arrival reads them through its own L2 (plain
// loads, the fast path) only when every arrival, itself included, ran on the
// XCD the tile map intended (blockIdx % 8, so all of them on one XCD and one
// L2); otherwise it reads them with device-coherent loads.  The device deals
// the workgroups of a launch to XCDs in blockIdx % 8 order only while nothing
// else uses the GPU in between (other queues' work, e.g. another library's
// kernels in the same process, and graph replays change the order), so the
// placement is checked per workgroup at run time and never assumed.
#pragma once
#include "qnn_internal.h"

namespace qnn {
namespace dev {

// Hardware XCC id of the executing wave (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() { return int(__builtin_amdgcn_s_getreg((3 << 11) | 20)) & 15; }

// The workgroup runs on the XCD the tile map intended (`local`: the context
// found the blockIdx % 8 dealing when it was created and is not capturing).
__device__ __forceinline__ bool on_home_xcd(int local) { return local && xcc_id() == int(blockIdx.x & 7); }

// Device-scope (write-through) store of an exchanged value.
__device__ __forceinline__ void xstore(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Load of an exchanged value: through this XCD's L2 when `l2` (every writer
// ran on this XCD), else device-coherent.
__device__ __forceinline__ float xload(const float *p, bool l2) {
  return l2 ? *p : __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Completes this wave's exchange stores, then takes a ticket; true (uniform)
// for the last of `arrivals` arrivals, which then owns the combine, reads with
// xload(p, l2) and resets the counter for the next launch.  A ticket counts 1
// per arrival plus 2^16 per arrival off its home XCD.
__device__ __forceinline__ bool last_arrival(unsigned *counter, unsigned arrivals, int lane, int local, bool &l2) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const bool home = on_home_xcd(local);
  unsigned ticket = 0;
  if (lane == 0)
    ticket = __hip_atomic_fetch_add(counter, home ? 1u : 1u + (1u << 16), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0);
  if ((ticket & 0xFFFFu) != arrivals - 1) return false;
  l2 = home && (ticket >> 16) == 0;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return true;
}
__device__ __forceinline__ void reset_counter(unsigned *counter, int lane) {
  if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// acc[m] = sum over s in slice order of part(s, m); PU independent loads per
// token in flight.
template <int MT, int PU, class AddrF>
__device__ __forceinline__ void sum_slices(float (&acc)[MT], AddrF part, int slices, bool l2) {
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
  for (int s0 = 0; s0 < slices; s0 += PU) {
    float v[PU][MT];
#pragma unroll
    for (int j = 0; j < PU; ++j)
      if (s0 + j < slices)
#pragma unroll
        for (int m = 0; m < MT; ++m) v[j][m] = xload(part(s0 + j, m), l2);
#pragma unroll
    for (int j = 0; j < PU; ++j)
      if (s0 + j < slices)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] += v[j][m];
  }
}

// blockIdx -> (unit, rest): every workgroup of a unit has the same
// blockIdx % 8, so with the blockIdx % 8 dealing the split-K partial sums of a
// unit stay in one L2.  `per` = workgroups per unit.
__device__ __forceinline__ bool map_tile(int b, int per, int units, int &unit, int &rest) {
  const int xcd = b & 7, k = b >> 3;
  const int q = k / per;
  unit = q * 8 + xcd;
  rest = k - q * per;
  return unit < units;
}

}  // namespace dev
}  // namespace qnn
