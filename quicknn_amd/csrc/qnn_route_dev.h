// qnn_route_dev.h -- GO_MOE_ROUTE's selection for one token row in one wave
// (moe.comp:25-50), shared by the route op (qnn_misc.hip) and the one-token
// MoE launch that computes its routes itself (qnn_moe.hip), so both give the
// same ids and probabilities bit for bit.
//
// The rule is the reference's: v_e = exp(l_e - max), denominator = the sum of
// the v_e, p_e = v_e / denominator, and experts are ranked by p (descending)
// with ties to the lower id.  Two distinct logits whose probabilities round
// to the same float therefore tie, and the lower id wins.
//  - exp is the correctly rounded fp32 exponential (computed in double, then
//    rounded once), so the value does not depend on a library's expf.
//  - The denominator is summed in the reference's order: 256 partial sums,
//    partial L over experts L, L+256, L+512, ... in ascending id, then the
//    tree partial[L] += partial[L + s] for s = 128, 64, ..., 1.  A lane of
//    this wave holds partials L = lane, lane+64, lane+128, lane+192.
//  - p = v / denominator is an IEEE division (correctly rounded).
//
// Up to 1024 experts: a lane holds J = experts/64 keys in registers, key =
// (bits of p) << 13 | (8191 - id) (p >= +0, so its bits order like its
// value), so a larger key is a larger probability, ties go to the lower id and
// all keys are distinct.  A 45-step binary search with wave ballots finds the
// k-th largest key T (count(key >= T) >= k, maximal); the k keys >= T are
// compacted to LDS and ranked against each other.  Renormalisation divides
// by the top-k sum taken in rank order.
#pragma once
#include "qnn_exchange.h"

namespace qnn {
namespace dev {

// exp(x) rounded once to fp32.
__device__ __forceinline__ float route_exp(float x) { return float(exp(double(x))); }

// The reference's denominator from this lane's four partial sums (partials
// lane, lane+64, lane+128, lane+192 of the 256): the tree over 256 partials,
// result broadcast from lane 0.
__device__ __forceinline__ float route_denominator(float q0, float q1, float q2, float q3) {
  q0 = q0 + q2;  // s = 128
  q1 = q1 + q3;
  float s = q0 + q1;  // s = 64
  // lanes < d hold the tree's values: lane i adds lane i + d = i ^ d
  s = s + xor_lanes<32>(s);
  s = s + xor_lanes<16>(s);
  s = s + xor_lanes<8>(s);
  s = s + xor_lanes<4>(s);
  s = s + xor_lanes<2>(s);
  s = s + xor_lanes<1>(s);
  return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(s)));
}

// The one-token MoE launch addresses its weights with the ids alone and
// finishes the probabilities (the top-k total) while its loads are in flight.
template <int J>
struct RouteRow {
  float pv;  // lane r < k: probability of the rank-r expert
  int id;    // lane r < k: the rank-r expert (descending probability, ties to the lower id)
};

// sel, ids, lvs: this wave's LDS scratch (64 each).
template <int J>
__device__ __forceinline__ void route_select(RouteRow<J> &r, const float *l, int experts, int k, int lane,
                                             unsigned long long *sel, int *ids, float *lvs) {
  float v[J];
  unsigned long long key[J];
  // one buffer load per key, all in flight together (past the row: zeros)
  const __amdgpu_buffer_rsrc_t lr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(l), 0, int(uint32_t(experts) * 4u), 0x00020000);
#pragma unroll
  for (int j = 0; j < J; ++j) v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(lr, (j * 64 + lane) * 4, 0, 0));
  float mx = -3.402823466e38f;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (j * 64 + lane < experts) mx = fmaxf(mx, v[j]);
  mx = wave_max_xor(mx);
  float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // partials lane + 64*i: experts (i + 4m)*64 + lane
#pragma unroll
  for (int j = 0; j < J; ++j) {
    v[j] = j * 64 + lane < experts ? route_exp(v[j] - mx) : 0.0f;
    q[j & 3] = q[j & 3] + v[j];
  }
  const float den = route_denominator(q[0], q[1], q[2], q[3]);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = j * 64 + lane;
    const float p = v[j] / den;
    key[j] = e < experts ? ((unsigned long long)__float_as_uint(p) << 13) | (unsigned long long)(8191 - e) : 0ull;
  }
  unsigned long long t = 0;  // the k-th largest key (real keys are > 0, and k <= experts)
  for (int b = 44; b >= 0; --b) {
    const unsigned long long cand = t | (1ull << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) cnt += __popcll(__ballot(key[j] >= cand));
    if (cnt >= k) t = cand;
  }
  int base = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool in = key[j] >= t;
    const unsigned long long bm = __ballot(in);
    if (in) sel[base + __popcll(bm & ((1ull << lane) - 1ull))] = key[j];
    base += __popcll(bm);
  }
  wave_lds_sync();
  const unsigned long long mine = lane < k ? sel[lane] : 0ull;
  int rank = 0;
  for (int m = 0; m < k; ++m) rank += sel[m] > mine;
  if (lane < k) {
    ids[rank] = 8191 - int(mine & 0x1FFFu);
    lvs[rank] = __uint_as_float(uint32_t(mine >> 13));
  }
  wave_lds_sync();
  r.id = lane < k ? ids[lane] : 0;
  r.pv = lane < k ? lvs[lane] : 0.0f;
}

// Lane r < k: probability of the rank-r expert (renormalised if normalize).
template <int J>
__device__ __forceinline__ float route_probs(const RouteRow<J> &r, int experts, int k, int normalize, int lane) {
  float total = 0.0f;
  for (int q = 0; q < k; ++q) total += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(r.pv), q));  // rank order
  return normalize ? r.pv / total : r.pv;
}

}  // namespace dev
}  // namespace qnn
