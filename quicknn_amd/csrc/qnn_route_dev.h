// qnn_route_dev.h -- GO_MOE_ROUTE's selection for one token row in one wave
// (moe.comp:25-50), shared by the route op (qnn_misc.hip) and the one-token
// MoE launch that computes its routes itself (qnn_moe.hip), so both give the
// same ids and probabilities bit for bit.
//
// Up to 1024 experts: a lane holds J = experts/64 keys in registers, key =
// (order-preserving bits of the logit) << 13 | (8191 - id), so a larger key is
// a larger logit, ties go to the lower id and all keys are distinct (-0 is
// keyed as +0, as the reference's comparisons treat them).  A 45-step binary
// search with wave ballots finds the k-th largest key T (count(key >= T) >= k,
// maximal); the k keys >= T are compacted to LDS and ranked against each
// other.  Probabilities: p = exp(l - max) / denominator with the denominator
// taken as each lane's experts in ascending id, then a butterfly sum broadcast
// from lane 0; renormalisation divides by the top-k sum in rank order.
#pragma once
#include "qnn_exchange.h"

namespace qnn {
namespace dev {

// Selection, then probabilities: the one-token MoE launch addresses its
// weights with the ids alone and computes the probabilities while its loads
// are in flight.  The probability phase uses no LDS and no barrier, so it
// does not hold up the waves that stage activations meanwhile.
template <int J>
struct RouteRow {
  float v[J];   // this lane's logits (experts j*64 + lane)
  float lv;     // lane r < k: logit of the rank-r expert
  float mx;     // the largest logit
  int id;       // lane r < k: the rank-r expert (descending logit, ties to the lower id)
};

// sel, ids, lvs: this wave's LDS scratch (64 each).
template <int J>
__device__ __forceinline__ void route_select(RouteRow<J> &r, const float *l, int experts, int k, int lane,
                                             unsigned long long *sel, int *ids, float *lvs) {
  unsigned long long key[J];
  // one buffer load per key, all in flight together (past the row: zeros)
  const __amdgpu_buffer_rsrc_t lr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(l), 0, int(uint32_t(experts) * 4u), 0x00020000);
#pragma unroll
  for (int j = 0; j < J; ++j) r.v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(lr, (j * 64 + lane) * 4, 0, 0));
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = j * 64 + lane;
    const uint32_t u = r.v[j] == 0.0f ? 0u : __float_as_uint(r.v[j]);
    const uint32_t m = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    key[j] = e < experts ? (((unsigned long long)m << 13) | (unsigned long long)(8191 - e)) : 0ull;
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
  const uint32_t mm = uint32_t(mine >> 13);
  if (lane < k) {
    ids[rank] = 8191 - int(mine & 0x1FFFu);
    lvs[rank] = __uint_as_float((mm & 0x80000000u) ? (mm & 0x7FFFFFFFu) : ~mm);
  }
  wave_lds_sync();
  r.id = lane < k ? ids[lane] : 0;
  r.lv = lane < k ? lvs[lane] : 0.0f;
  r.mx = lvs[0];
}

// Lane r < k: probability of the rank-r expert (renormalised if normalize).
template <int J>
__device__ __forceinline__ float route_probs(const RouteRow<J> &r, int experts, int k, int normalize, int lane) {
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (j * 64 + lane < experts) part += expf(r.v[j] - r.mx);
  for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
  const float denominator = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(part)));  // lane 0's
  const float p = lane < k ? expf(r.lv - r.mx) / denominator : 0.0f;
  float total = 0.0f;
  for (int q = 0; q < k; ++q) total += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(p), q));  // rank order
  return normalize ? p / total : p;
}

}  // namespace dev
}  // namespace qnn
