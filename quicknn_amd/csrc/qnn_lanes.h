// qnn_lanes.h -- cross-lane exchange of one wave without the LDS crossbar.
//
// xor_lanes<OFF>(x) returns x of lane (lane ^ OFF), as __shfl_xor(x, OFF)
// does for a full 64-lane wave, but on the VALU: DPP quad permutes (OFF 1, 2),
// DPP row shifts (4) and rotates (8), and gfx950's v_permlane16_swap /
// v_permlane32_swap (16, 32).  __shfl_xor goes through ds_bpermute, whose
// latency sits on every step of a butterfly reduction.  Only data moves, so a
// reduction keeps its exact pairing order and its result.
#pragma once
#include <hip/hip_runtime.h>

namespace qnn {
namespace dev {

template <int OFF>
__device__ __forceinline__ int xor_lanes_i(int v) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane xor");
  if constexpr (OFF == 1) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (OFF == 2) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (OFF == 4) {
    const int lo = __builtin_amdgcn_mov_dpp(v, 0x114, 0xF, 0xF, false);  // row_shr:4 -> lane - 4
    const int hi = __builtin_amdgcn_mov_dpp(v, 0x104, 0xF, 0xF, false);  // row_shl:4 -> lane + 4
    return (__lane_id() & 4) ? lo : hi;
  } else if constexpr (OFF == 8) {
    return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);  // row_ror:8 in 16-lane rows
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(unsigned(v), unsigned(v), false, false);
    return int((__lane_id() & 16) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(unsigned(v), unsigned(v), false, false);
    return int((__lane_id() & 32) ? r[0] : r[1]);
  }
}
template <int OFF>
__device__ __forceinline__ float xor_lanes(float x) {
  return __int_as_float(xor_lanes_i<OFF>(__float_as_int(x)));
}

// The full-wave butterflies of __shfl_xor(x, 32), (.., 16), .., (.., 1), in
// that order: every lane ends with the wave's maximum or sum.
__device__ __forceinline__ float wave_max_xor(float x) {
  x = fmaxf(x, xor_lanes<32>(x));
  x = fmaxf(x, xor_lanes<16>(x));
  x = fmaxf(x, xor_lanes<8>(x));
  x = fmaxf(x, xor_lanes<4>(x));
  x = fmaxf(x, xor_lanes<2>(x));
  return fmaxf(x, xor_lanes<1>(x));
}
__device__ __forceinline__ float wave_sum_xor(float x) {
  x += xor_lanes<32>(x);
  x += xor_lanes<16>(x);
  x += xor_lanes<8>(x);
  x += xor_lanes<4>(x);
  x += xor_lanes<2>(x);
  return x + xor_lanes<1>(x);
}

}  // namespace dev
}  // namespace qnn
