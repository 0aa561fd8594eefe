// qnn_misc.hip -- small ops on the decode path: fill, add, SwiGLU/GEGLU,
// finite check, RMS/LayerNorm, MoE route, gather and scatter.  Semantics
// follow the Vulkan shaders cited per kernel.
#include "qnn_int4_dev.h"
#include "qnn_route_dev.h"

namespace qnn {
namespace {

__device__ __forceinline__ float silu_dev(float x) {  // tensor.comp:22
  return x >= 20.0f ? x : (x <= -20.0f ? 0.0f : x / (1.0f + expf(-x)));
}
__device__ __forceinline__ float gelu_dev(float x) {  // tensor.comp:23 (tanh approximation)
  return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float load_vec(const void *p, int bf16, int i) {
  if (bf16) return __uint_as_float(uint32_t(static_cast<const uint16_t *>(p)[i]) << 16);
  return static_cast<const float *>(p)[i];
}

__global__ void k_fill(float *dst, int n, uint32_t bits) {  // tensor.comp:219 (GO_FILL)
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = __uint_as_float(bits);
}

// GO_ADD (tensor.comp:221): dst[doff + r*stride + j] += alpha * a[soff + id], r = id / cols.
__global__ void k_add(float *dst, const float *a, int n, int cols, int stride, float alpha, int doff, int soff) {
  int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  int r = id / cols, j = id % cols;
  size_t t = size_t(doff) + size_t(r) * stride + j;
  dst[t] = dst[t] + alpha * a[soff + id];
}

// GO_SWIGLU / GO_GEGLU (tensor.comp:228).
__global__ void k_glu(float *dst, const float *a, const float *b, int n, int inter, int interleaved, int gelu) {
  int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  if (interleaved) {
    int r = id / inter, j = id % inter;
    dst[id] = silu_dev(a[size_t(r) * 2 * inter + j]) * a[size_t(r) * 2 * inter + inter + j];
  } else {
    dst[id] = (gelu ? gelu_dev(a[id]) : silu_dev(a[id])) * b[id];
  }
}

// GO_FINITE (tensor.comp:235): OR 1 into the error word on NaN/Inf.
__global__ void k_finite(const float *a, int n, int *flag) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  bool bad = false;
  if (i < n) {
    float x = a[i];
    bad = isnan(x) || isinf(x);
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(flag, 1);
}

// GO_NORM (tensor.comp:63-73), row-major rows: optional mean subtraction
// (flags&1), x*inversesqrt(mean(x^2)+eps)*(gamma|1 [+1 if flags&4]) [+beta].
__global__ __launch_bounds__(256) void k_norm(float *dst, const float *a, const void *gamma, int gamma_bf16,
                                              const void *beta, int beta_bf16, int dim, int flags, int soff,
                                              int unit_gamma, float eps) {
  __shared__ float red[256];
  const int row = blockIdx.x, lane = threadIdx.x;
  const float *x = a + soff + size_t(row) * dim;
  auto sum_group = [&](float v) {
    red[lane] = v;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if (lane < s) red[lane] += red[lane + s];
      __syncthreads();
    }
    float r = red[0];
    __syncthreads();
    return r;
  };
  float mean = 0.0f, part = 0.0f;
  if (flags & 1) {
    for (int j = lane; j < dim; j += 256) part += x[j];
    mean = sum_group(part) / float(dim);
  }
  part = 0.0f;
  for (int j = lane; j < dim; j += 256) {
    float v = x[j] - mean;
    part += v * v;
  }
  const float squares = sum_group(part);
  const float inv = rsqrtf(squares / float(dim) + eps);
  for (int j = lane; j < dim; j += 256) {
    float scale = (unit_gamma ? 1.0f : load_vec(gamma, gamma_bf16, j)) + ((flags & 4) ? 1.0f : 0.0f);
    float b = ((flags & 1) && !(flags & 8) && beta) ? load_vec(beta, beta_bf16, j) : 0.0f;
    dst[soff + size_t(row) * dim + j] = (x[j] - mean) * inv * scale + b;
  }
}

// GO_MOE_ROUTE (moe.comp:25-50): fp32 softmax, exact top-k by probability
// with ties to the lower id, optional renormalisation by the rank-ordered
// top-k sum.  exp is rounded once from double and the denominator is summed in
// the reference's 256-partial order (qnn_route_dev.h), so ids and
// probabilities match the CPU oracle bit for bit.  One wave per token row;
// two selection methods with the same result:
//
// * up to 1024 experts (k_moe_route_reg): keys in registers and a ballot
//   radix select (dev::route_select, qnn_route_dev.h).
// * more experts (k_moe_route): probabilities in LDS; each of the k rounds is
//   a scan of the lane's experts plus a 6-step butterfly argmax over
//   (probability desc, id asc), a strict total order, so every lane agrees on
//   the winner.
template <int J>
__global__ __launch_bounds__(64) void k_moe_route_reg(float *routes, const float *logits, int rows, int experts, int k,
                                                      int normalize) {
  __shared__ unsigned long long sel[64];
  __shared__ int ids[64];
  __shared__ float lvs[64];
  const int row = blockIdx.x, lane = threadIdx.x;
  dev::RouteRow<J> r;
  dev::route_select<J>(r, logits + size_t(row) * experts, experts, k, lane, sel, ids, lvs);
  const float p = dev::route_probs<J>(r, experts, k, normalize, lane);
  if (lane < k) {
    const int target = row * k + lane;
    routes[target] = __uint_as_float(uint32_t(r.id));
    routes[size_t(rows) * k + target] = p;
  }
}

constexpr int kRouteNone = 0x7fffffff;
__device__ __forceinline__ bool route_better(float v, int i, float bv, int bi) {
  return i != kRouteNone && (bi == kRouteNone || v > bv || (v == bv && i < bi));
}
__global__ __launch_bounds__(64) void k_moe_route(float *routes, const float *logits, int rows, int experts, int k,
                                                  int normalize) {
  extern __shared__ float sh[];  // experts probabilities, then experts "taken" bytes
  float *pr = sh;
  uint8_t *taken = reinterpret_cast<uint8_t *>(sh + experts);
  const int row = blockIdx.x, lane = threadIdx.x;
  const float *l = logits + size_t(row) * experts;
  float mx = -3.402823466e38f;
  for (int e = lane; e < experts; e += 64) {
    const float v = l[e];
    pr[e] = v;
    taken[e] = 0;
    mx = fmaxf(mx, v);
  }
  mx = dev::wave_max_xor(mx);
  // The lane's own LDS entries: partial lane + 64*i sums experts lane + 64*i + 256*m, ascending m.
  float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = 0; i < 4; ++i)
    for (int e = lane + 64 * i; e < experts; e += 256) {
      const float v = dev::route_exp(pr[e] - mx);
      pr[e] = v;
      q[i] = q[i] + v;
    }
  const float den = dev::route_denominator(q[0], q[1], q[2], q[3]);
  for (int e = lane; e < experts; e += 64) pr[e] = pr[e] / den;
  __syncthreads();
  int my_id = 0;
  float my_p = 0.0f;
  for (int r = 0; r < k; ++r) {
    float best = -INFINITY;
    int bid = kRouteNone;
    for (int e = lane; e < experts; e += 64) {
      const float v = pr[e];
      if (!taken[e] && route_better(v, e, best, bid)) {
        best = v;
        bid = e;
      }
    }
    auto step = [&](auto off) {  // the butterfly of __shfl_xor(., 32 .. 1), on the VALU
      constexpr int O = decltype(off)::value;
      const float ov = dev::xor_lanes<O>(best);
      const int oi = dev::xor_lanes_i<O>(bid);
      if (route_better(ov, oi, best, bid)) {
        best = ov;
        bid = oi;
      }
    };
    step(std::integral_constant<int, 32>());
    step(std::integral_constant<int, 16>());
    step(std::integral_constant<int, 8>());
    step(std::integral_constant<int, 4>());
    step(std::integral_constant<int, 2>());
    step(std::integral_constant<int, 1>());
    bid = __builtin_amdgcn_readfirstlane(bid);  // lane 0's; k <= experts: a candidate always exists
    if (lane == 0) taken[bid] = 1;
    if (lane == r) {
      my_id = bid;
      my_p = pr[bid];
    }
    __syncthreads();
  }
  float total = 0.0f;
  for (int r = 0; r < k; ++r) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), r));  // rank order
  if (lane < k) {
    const int target = row * k + lane;
    routes[target] = __uint_as_float(uint32_t(my_id));
    routes[size_t(rows) * k + target] = normalize ? my_p / total : my_p;
  }
}

// GO_MOE_GATHER (moe.comp:124).  Dispatch indices come from the caller: one
// that points outside src/dst is reported (error bit 16), never dereferenced.
__global__ void k_moe_gather(float *dst, const float *src, size_t src_n, const float *indices, int n, int hidden,
                             int topk, int offset, int *err) {
  int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  int r = id / hidden, j = id % hidden;
  uint32_t route = __float_as_uint(indices[offset + r]);
  const size_t si = size_t(route / topk) * hidden + j;
  if (si < src_n) {
    dst[id] = src[si];
  } else {
    dst[id] = 0.0f;
    atomicOr(err, 16);
  }
}

// GO_MOE_SCATTER (moe.comp:125-126).
__global__ void k_moe_scatter(float *dst, size_t dst_n, const float *y, const float *indices, const float *routes,
                              size_t routes_n, int n, int hidden, int topk, int offset, int route_index,
                              int single_row, int prob_base, int *err) {
  int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  int r = id / hidden, j = id % hidden;
  uint32_t route = single_row ? uint32_t(route_index) : __float_as_uint(indices[offset + r]);
  size_t target = size_t(route / topk) * hidden + j;
  const size_t pi = size_t(prob_base) + route;
  if (target >= dst_n || pi >= routes_n) {
    atomicOr(err, 16);
    return;
  }
  dst[target] = add_mul_nofma(dst[target], y[id], routes[pi]);
}

// Bias after a projection (GO_CONV_OUTPUT with bias in Linear, Implementation.inc:848-849, :892-893).
__global__ void k_bias_add(float *dst, const void *bias, int bf16, int rows, int cols) {
  int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * cols) return;
  dst[id] = dst[id] + load_vec(bias, bf16, id % cols);
}

// Rows of `cols` floats -> rows of `cols_pad` floats, zero tail.
__global__ void k_pad_rows(float *dst, const float *src, int rows, int cols, int cols_pad) {
  const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (long long)rows * cols_pad) return;
  const int r = int(id / cols_pad), c = int(id % cols_pad);
  dst[id] = c < cols ? src[(long long)r * cols + c] : 0.0f;
}

// Records the hardware XCC id (HW_REG_XCC_ID) of each workgroup.
inline int blocks(long long n, int t) { return int((n + t - 1) / t); }

// Plain stream of n16 16-byte pieces (diagnostic: the HBM stream floor the
// matvec kernels are measured against).  The same loads as their weight
// stream: non-temporal raw buffer loads, every piece requested at once (each
// thread issues its U loads before using any); one store per launch at most,
// on a condition that depends on every byte, so no load can be dropped.
constexpr int kStreamU = 8;
__global__ __launch_bounds__(256) void k_stream_read(const void *src, uint32_t n16, uint32_t *out) {
  const auto r = dev::rsrc(src, size_t(n16) * 16);
  const uint32_t base = (blockIdx.x * 256u + threadIdx.x) * 16u;
  const uint32_t stride = gridDim.x * 256u * 16u;
  uint4 v[kStreamU];
#pragma unroll
  for (int i = 0; i < kStreamU; ++i) v[i] = dev::ld128<dev::kStream>(r, base, uint32_t(i) * stride);
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < kStreamU; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (acc == 0x9E3779B9u) out[0] = acc;
}

}  // namespace

void misc_stream_read(const void *src, size_t bytes, uint32_t *out, hipStream_t s) {
  const uint32_t n16 = uint32_t(bytes / 16);
  const uint32_t per_wg = 256u * kStreamU;
  hipLaunchKernelGGL(k_stream_read, dim3((n16 + per_wg - 1) / per_wg), dim3(256), 0, s, src, n16, out);
}

void misc_fill(float *dst, int n, uint32_t bits, hipStream_t s) {
  hipLaunchKernelGGL(k_fill, dim3(blocks(n, 256)), dim3(256), 0, s, dst, n, bits);
  hip_check(hipGetLastError(), "fill");
}
void misc_add(float *dst, const float *a, int n, int cols, int dst_stride, float alpha, int dst_off, int src_off,
              hipStream_t s) {
  hipLaunchKernelGGL(k_add, dim3(blocks(n, 256)), dim3(256), 0, s, dst, a, n, cols, dst_stride, alpha, dst_off,
                     src_off);
  hip_check(hipGetLastError(), "add");
}
void misc_glu(float *dst, const float *a, const float *b, int n, int inter, int interleaved, int gelu,
              hipStream_t s) {
  hipLaunchKernelGGL(k_glu, dim3(blocks(n, 256)), dim3(256), 0, s, dst, a, b, n, inter, interleaved, gelu);
  hip_check(hipGetLastError(), "glu");
}
void misc_finite(const float *a, int n, int *flag, hipStream_t s) {
  hipLaunchKernelGGL(k_finite, dim3(blocks(n, 256)), dim3(256), 0, s, a, n, flag);
  hip_check(hipGetLastError(), "finite");
}
void misc_norm(float *dst, const float *a, const void *gamma, int gamma_bf16, const void *beta, int beta_bf16,
               int rows, int dim, int flags, int src_off, int unit_gamma, float eps, hipStream_t s) {
  hipLaunchKernelGGL(k_norm, dim3(rows), dim3(256), 0, s, dst, a, gamma, gamma_bf16, beta, beta_bf16, dim, flags,
                     src_off, unit_gamma, eps);
  hip_check(hipGetLastError(), "norm");
}
void misc_moe_route(float *routes, const float *logits, int rows, int experts, int k, int normalize,
                    hipStream_t s) {
  const int j = (experts + 63) / 64;
  if (j <= 1) hipLaunchKernelGGL(k_moe_route_reg<1>, dim3(rows), dim3(64), 0, s, routes, logits, rows, experts, k, normalize);
  else if (j <= 2) hipLaunchKernelGGL(k_moe_route_reg<2>, dim3(rows), dim3(64), 0, s, routes, logits, rows, experts, k, normalize);
  else if (j <= 4) hipLaunchKernelGGL(k_moe_route_reg<4>, dim3(rows), dim3(64), 0, s, routes, logits, rows, experts, k, normalize);
  else if (j <= 8) hipLaunchKernelGGL(k_moe_route_reg<8>, dim3(rows), dim3(64), 0, s, routes, logits, rows, experts, k, normalize);
  else if (j <= 16) hipLaunchKernelGGL(k_moe_route_reg<16>, dim3(rows), dim3(64), 0, s, routes, logits, rows, experts, k, normalize);
  else hipLaunchKernelGGL(k_moe_route, dim3(rows), dim3(64), size_t(experts) * 5, s, routes, logits, rows, experts, k, normalize);
  hip_check(hipGetLastError(), "moe route");
}
void misc_moe_gather(float *dst, const float *src, size_t src_n, const float *indices, int n, int hidden, int topk,
                     int offset, int *err, hipStream_t s) {
  hipLaunchKernelGGL(k_moe_gather, dim3(blocks(n, 256)), dim3(256), 0, s, dst, src, src_n, indices, n, hidden, topk,
                     offset, err);
  hip_check(hipGetLastError(), "moe gather");
}
void misc_moe_scatter(float *dst, size_t dst_n, const float *y, const float *indices, const float *routes,
                      size_t routes_n, int n, int hidden, int topk, int offset, int route_index, int single_row,
                      int prob_base, int *err, hipStream_t s) {
  hipLaunchKernelGGL(k_moe_scatter, dim3(blocks(n, 256)), dim3(256), 0, s, dst, dst_n, y, indices, routes, routes_n,
                     n, hidden, topk, offset, route_index, single_row, prob_base, err);
  hip_check(hipGetLastError(), "moe scatter");
}
void misc_bias_add(float *dst, const void *bias, int bias_bf16, int rows, int cols, hipStream_t s) {
  hipLaunchKernelGGL(k_bias_add, dim3(blocks((long long)rows * cols, 256)), dim3(256), 0, s, dst, bias, bias_bf16,
                     rows, cols);
  hip_check(hipGetLastError(), "bias add");
}

void misc_pad_rows(float *dst, const float *src, int rows, int cols, int cols_pad, hipStream_t s) {
  hipLaunchKernelGGL(k_pad_rows, dim3(blocks((long long)rows * cols_pad, 256)), dim3(256), 0, s, dst, src, rows, cols,
                     cols_pad);
  hip_check(hipGetLastError(), "pad rows");
}

}  // namespace qnn
