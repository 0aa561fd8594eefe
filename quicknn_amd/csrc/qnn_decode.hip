// qnn_decode.hip -- the rest of a resident decode layer: RoPE, KV-cache
// append, cached attention, seen-token flags and token sampling.
//
// Semantics follow the Vulkan shaders cited per kernel
// (src/backends/vulkan/shaders/tensor.comp, attention.comp) and the host
// methods that drive them (QuickNN.Vulkan.Context.Implementation.inc).
//
// Cached attention is split over keys (flash-decoding): a workgroup owns one
// query row, a batch of the query heads that share one KV head (so K and V are
// read once for all of them), and a chunk of keys; it writes the chunk's
// running max, sum and unnormalised output, and a second launch merges the
// chunks.  The KV cache is fp32 in the reference's layout: K transposed
// [kv_heads][dim][capacity] (keys contiguous, coalesced score loads), then V
// [kv_heads][capacity][dim] (channels contiguous).
//
// Sampling is one launch: workgroups take exact local top-k of 4096-token
// tiles, and the last workgroup to arrive merges the tiles' candidates, takes
// the global top-k and draws the token, as tensor.comp:123-199 does in two.
#include <cmath>

#include "qnn_exchange.h"
#include "qnn_lanes.h"

namespace qnn {
namespace {

// ---------------------------------------------------------------------------
// GO_LLM_ROPE (tensor.comp:318-327): rotate the pairs (j, j + dim/2) of each
// head row by angle (position + row) * theta^(-2j/dim).  The angle, its sine
// and cosine and the rotation are evaluated in double and rounded once, as the
// reference's CPU statement of the same rotation does
// (src/models/QuickNN.Models.QwenHybrid.CPU.pas:51-67).
__global__ void k_rope(float *dst, const float *src, int n, int heads, int dim, int position, float theta) {
#pragma clang fp contract(off)
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  const int half = dim / 2, j = id % half, hr = id / half, r = hr / heads;
  const double angle = double(position + r) * pow(double(theta), -2.0 * double(j) / double(dim));
  double s, c;
  sincos(angle, &s, &c);
  const size_t x = size_t(hr) * dim + j, y = x + half;
  const double a = src[x], b = src[y];
  dst[x] = float(a * c - b * s);
  dst[y] = float(a * s + b * c);
}

// GO_LLM_CACHE_WRITE (tensor.comp:313-317): append rows of K and V at
// position + row: K transposed, V head-major.
__global__ void k_cache_write(float *cache, const float *k, const float *v, int n, int kv_heads, int dim, int cap,
                              int position) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  const int width = kv_heads * dim, r = id / width, h = (id % width) / dim, j = id % dim, t = position + r;
  cache[(size_t(h) * dim + j) * cap + t] = k[id];
  cache[size_t(cap) * width + (size_t(h) * cap + t) * dim + j] = v[id];
}

// GO_LLM_SEEN (tensor.comp:328): flag[token] |= 1 for each token id below vocab.
__global__ void k_seen(unsigned *flags, const unsigned *ids, int n, unsigned vocab) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  const unsigned token = ids[id];
  if (token < vocab) atomicOr(&flags[token], 1u);
}

// GO_SCALE (tensor.comp:309): x * a + b.  GO_SOFTCAP (tensor.comp:308):
// cap * tanh(clamp(x / cap, -20, 20)).
__global__ void k_scale(float *dst, const float *src, int n, float a, float b) {
#pragma clang fp contract(off)
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id < n) dst[id] = src[id] * a + b;
}
__global__ void k_softcap(float *dst, const float *src, int n, float cap) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id < n) dst[id] = cap * tanhf(fminf(fmaxf(src[id] / cap, -20.0f), 20.0f));
}

// Gather (Context.Implementation.inc:1228-1267; tensor.comp:245-251): rows
// of an F32, BF16 or int8 (times a per-row F32 scale) table by token id (raw
// bits); ids at or past the vocabulary give zeros.
__global__ void k_gather(float *out, const unsigned *ids, const void *w, int kind, const float *scales, int n, int dim,
                         int vocab) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  const int r = id / dim, j = id % dim;
  const unsigned token = ids[r];
  if (token >= unsigned(vocab)) {
    out[id] = 0.0f;
    return;
  }
  const size_t index = size_t(token) * dim + j;
  float x;
  if (kind == 1)
    x = __uint_as_float(uint32_t(static_cast<const uint16_t *>(w)[index]) << 16);
  else if (kind == 2)
    x = float(static_cast<const int8_t *>(w)[index]) * scales[token];
  else
    x = static_cast<const float *>(w)[index];
  out[id] = x;
}

// ---------------------------------------------------------------------------
// Cached attention (attention.comp, the online path the resident context
// dispatches with mask mode 2, or 4 with a per-row key mask).
//
// A workgroup owns (query row, GB heads of one KV head, a chunk of keys).  It
// walks the chunk in sub-chunks of up to 256 keys with an online softmax.
// Score pass: P = 256 / sub-chunk threads per key, each over dim / P channels
// with up to 32 independent K loads in flight (K^T rows are contiguous in the
// key, so a wave's load covers 64 consecutive keys).  Value pass: float4
// channel groups, dim / 4 lanes per key and 256 / (dim / 4) keys at a time,
// four or eight keys' loads in flight per lane.
constexpr int kAttnThreads = 256;
constexpr int kAttnSub = 256;  // keys per sub-chunk at most

struct AttnArgs {
  int rows, cap, heads, kv_heads, dim, position, window, masked;
  float softcap, scale;
  int group, gpk, splits, chunk, sub, parts, lpk, kl, nd4;
};

__device__ __forceinline__ void key_range(const AttnArgs &a, int r, int &start, int &end) {
  end = a.position + r + 1;
  start = (a.window > 0 && end > a.window) ? end - a.window : 0;
}

// Four channels c .. c+3 of a row of `dim` floats: one 16-byte access when
// rows are 16-byte aligned (dim % 4 == 0), else element by element within dim.
__device__ __forceinline__ float4 load4(const float *row, int c, int dim) {
  if ((dim & 3) == 0) return *reinterpret_cast<const float4 *>(row + c);
  return make_float4(row[c], c + 1 < dim ? row[c + 1] : 0.f, c + 2 < dim ? row[c + 2] : 0.f,
                     c + 3 < dim ? row[c + 3] : 0.f);
}
// Cache reads: each K and V element is read once per call, so they stream
// (non-temporal; 32k keys 60.8 -> 57.0 us) and leave the L2 to q and the
// chunk partials.
__device__ __forceinline__ float kvload(const float *p) { return __builtin_nontemporal_load(p); }
typedef float kv_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load4v(const float *row, int c, int dim) {
  if ((dim & 3) == 0) {
    const kv_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const kv_f32x4 *>(row + c));
    return make_float4(v.x, v.y, v.z, v.w);
  }
  return load4(row, c, dim);
}
__device__ __forceinline__ void store4(float *row, int c, int dim, float4 v) {
  if ((dim & 3) == 0) {
    *reinterpret_cast<float4 *>(row + c) = v;
    return;
  }
  row[c] = v.x;
  if (c + 1 < dim) row[c + 1] = v.y;
  if (c + 2 < dim) row[c + 2] = v.z;
  if (c + 3 < dim) row[c + 3] = v.w;
}

template <int GB>
__device__ __forceinline__ void block_max_sum(float (&v)[GB], float *red, bool is_max) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const float x = is_max ? dev::wave_max_xor(v[g]) : dev::wave_sum_xor(v[g]);
    if (lane == 0) red[g * 4 + wave] = x;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < GB; ++g)
    v[g] = is_max ? fmaxf(fmaxf(red[g * 4], red[g * 4 + 1]), fmaxf(red[g * 4 + 2], red[g * 4 + 3]))
                  : (red[g * 4] + red[g * 4 + 1]) + (red[g * 4 + 2] + red[g * 4 + 3]);
  __syncthreads();
}

template <int GB, int ND4>
__global__ __launch_bounds__(kAttnThreads) void k_attn(const float *__restrict__ q, const float *__restrict__ cache,
                                                       float *__restrict__ out, float *__restrict__ opart,
                                                       float *__restrict__ mlpart, AttnArgs a) {
  extern __shared__ float lds[];
  float *qs = lds;                        // [GB][dim]
  float *ps = qs + GB * a.dim;            // [GB][sub]
  float *red = ps + GB * kAttnSub;        // [GB][4]
  float *xred = red + GB * 4;             // score parts [parts][GB][sub], then value lanes [kl][GB][dim]
  const int tid = threadIdx.x;
  const int kh = blockIdx.x / a.gpk, h0 = kh * a.group + (blockIdx.x % a.gpk) * GB;
  const int r = blockIdx.y, s = blockIdx.z;
  int start, end;
  key_range(a, r, start, end);
  const int k0 = start + s * a.chunk, k1 = min(end, k0 + a.chunk);
  const size_t width = size_t(a.kv_heads) * a.dim;
  const float *kt = cache + size_t(kh) * a.dim * a.cap;
  const float *vb = cache + size_t(a.cap) * width + size_t(kh) * a.cap * a.dim;
  const unsigned *mask = reinterpret_cast<const unsigned *>(cache + 2 * size_t(a.cap) * width) + size_t(r) * a.cap;

  // q rows of the batch: GB * dim <= 8 * 1152 floats, at most 36 per thread,
  // loaded before any is stored so they are in flight together.
  {
    constexpr int QMAX = (GB * 1152 + kAttnThreads - 1) / kAttnThreads;
    float qv[QMAX];
#pragma unroll
    for (int u = 0; u < QMAX; ++u) {
      const int i = tid + u * kAttnThreads;
      qv[u] = i < GB * a.dim ? q[(size_t(r) * a.heads + h0 + i / a.dim) * a.dim + i % a.dim] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < QMAX; ++u) {
      const int i = tid + u * kAttnThreads;
      if (i < GB * a.dim) qs[i] = qv[u];
    }
  }
  __syncthreads();

  const float mul = a.scale > 0.0f ? a.scale : 1.0f / sqrtf(float(a.dim));
  float m_run[GB], l_run[GB];
  float4 acc[GB][ND4];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < ND4; ++i) acc[g][i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int key_t = tid % a.sub, part = tid / a.sub;
  const int dp = (a.dim + a.parts - 1) / a.parts, d0 = part * dp, d1 = min(a.dim, d0 + dp);
  const int kk = tid / a.lpk, c4 = tid % a.lpk;  // value pass: key lane, float4 channel group

  constexpr int U = GB * ND4 >= 8 ? 4 : 8;
  auto load_values = [&](float4 (&vv)[U][ND4], int c0, int nkeys, int key0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key = key0 + u * a.kl;
#pragma unroll
      for (int i = 0; i < ND4; ++i) {
        const int cg = c4 + i * a.lpk;
        vv[u][i] = (kk < a.kl && key < nkeys && i < a.nd4 && cg * 4 < a.dim)
                       ? load4v(vb + size_t(c0 + key) * a.dim, cg * 4, a.dim)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  for (int c0 = k0; c0 < k1; c0 += a.sub) {
    const int c1 = min(k1, c0 + a.sub);
    // The first batch of V rows does not depend on the scores: request it
    // now, so it travels with the K loads below.
    float4 vfirst[U][ND4];
    load_values(vfirst, c0, c1 - c0, kk);
    // ---- scores (part of the channels per thread)
    const int j = c0 + key_t;
    bool valid = j < c1 && part < a.parts;
    if (valid && a.masked) valid = mask[j] != 0u;
    float sc[GB];
#pragma unroll
    for (int g = 0; g < GB; ++g) sc[g] = 0.0f;
    if (valid) {
      const float *kc = kt + j;
      int d = d0;
      for (; d + 32 <= d1; d += 32) {
        float kv[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) kv[u] = kvload(kc + size_t(d + u) * a.cap);
#pragma unroll
        for (int u = 0; u < 32; ++u)
#pragma unroll
          for (int g = 0; g < GB; ++g) sc[g] += qs[g * a.dim + d + u] * kv[u];
      }
      for (; d + 8 <= d1; d += 8) {
        float kv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) kv[u] = kvload(kc + size_t(d + u) * a.cap);
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int g = 0; g < GB; ++g) sc[g] += qs[g * a.dim + d + u] * kv[u];
      }
      for (; d < d1; ++d) {
        const float kv = kvload(kc + size_t(d) * a.cap);
#pragma unroll
        for (int g = 0; g < GB; ++g) sc[g] += qs[g * a.dim + d] * kv;
      }
    }
    if (a.parts > 1) {
#pragma unroll
      for (int g = 0; g < GB; ++g) xred[(part * GB + g) * a.sub + key_t] = sc[g];
      __syncthreads();
      if (part == 0)
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          float v = sc[g];
          for (int p = 1; p < a.parts; ++p) v += xred[(p * GB + g) * a.sub + key_t];
          sc[g] = v;
        }
      if (a.sub != 64) __syncthreads();
      valid = valid && part == 0;
    }
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float v = sc[g] * mul;
      if (a.softcap > 0.0f) v = a.softcap * tanhf(fminf(fmaxf(v / a.softcap, -20.0f), 20.0f));
      sc[g] = v;
    }
    float keep[GB];
    if (a.sub == 64) {
      // A 64-key sub-chunk: after the channel parts meet, wave 0 holds every
      // score (one key per lane) and runs the online softmax with wave
      // reductions; the other waves read the rescale factors from LDS.
      if (part == 0) {
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          const float mx = dev::wave_max_xor(valid ? sc[g] : -INFINITY);
          const float m_new = fmaxf(m_run[g], mx);
          keep[g] = m_new == -INFINITY ? 1.0f : expf(m_run[g] - m_new);
          const float p = (valid && m_new > -INFINITY) ? expf(sc[g] - m_new) : 0.0f;
          ps[g * kAttnSub + key_t] = p;
          const float ls = dev::wave_sum_xor(p);
          l_run[g] = l_run[g] * keep[g] + ls;
          m_run[g] = m_new;
          if (key_t == 0) {
            red[g] = keep[g];
            red[GB + g] = l_run[g];
            red[2 * GB + g] = m_run[g];
          }
        }
      }
      __syncthreads();  // publishes ps and the running state
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        keep[g] = red[g];
        l_run[g] = red[GB + g];
        m_run[g] = red[2 * GB + g];
      }
    } else {
      float cm[GB];
#pragma unroll
      for (int g = 0; g < GB; ++g) cm[g] = valid ? sc[g] : -INFINITY;
      block_max_sum<GB>(cm, red, true);
      float m_new[GB], ls[GB];
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        m_new[g] = fmaxf(m_run[g], cm[g]);
        keep[g] = m_new[g] == -INFINITY ? 1.0f : expf(m_run[g] - m_new[g]);
        const float p = (valid && m_new[g] > -INFINITY) ? expf(sc[g] - m_new[g]) : 0.0f;
        if (part == 0) ps[g * kAttnSub + key_t] = p;
        ls[g] = p;
      }
      block_max_sum<GB>(ls, red, false);  // its barriers also publish ps
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        l_run[g] = l_run[g] * keep[g] + ls[g];
        m_run[g] = m_new[g];
      }
    }
#pragma unroll
    for (int g = 0; g < GB; ++g) {
#pragma unroll
      for (int i = 0; i < ND4; ++i) {
        acc[g][i].x *= keep[g];
        acc[g][i].y *= keep[g];
        acc[g][i].z *= keep[g];
        acc[g][i].w *= keep[g];
      }
    }
    // ---- values: lane group kk walks keys kk, kk + kl, ..., U at a time
    if (kk < a.kl) {
      const int nkeys = c1 - c0;
      for (int key0 = kk; key0 < nkeys; key0 += U * a.kl) {
        float4 vv[U][ND4];
        if (key0 == kk) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < ND4; ++i) vv[u][i] = vfirst[u][i];
        } else {
          load_values(vv, c0, nkeys, key0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int key = key0 + u * a.kl;
          if (key < nkeys)
#pragma unroll
            for (int g = 0; g < GB; ++g) {
              const float w = ps[g * kAttnSub + key];
#pragma unroll
              for (int i = 0; i < ND4; ++i) {
                acc[g][i].x += w * vv[u][i].x;
                acc[g][i].y += w * vv[u][i].y;
                acc[g][i].z += w * vv[u][i].z;
                acc[g][i].w += w * vv[u][i].w;
              }
            }
        }
      }
    }
    __syncthreads();  // ps is rewritten by the next sub-chunk
  }

  // Sum the key lanes.
  if (a.kl > 1 && a.lpk == 32) {
    // Two key lanes per wave (lanes 0-31 and 32-63): they meet by a lane
    // shuffle, then the four waves' sums in LDS.
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
      for (int i = 0; i < ND4; ++i) {
        acc[g][i].x += dev::xor_lanes<32>(acc[g][i].x);  // lanes 0-31 take 32-63 (the upper sums are unused)
        acc[g][i].y += dev::xor_lanes<32>(acc[g][i].y);
        acc[g][i].z += dev::xor_lanes<32>(acc[g][i].z);
        acc[g][i].w += dev::xor_lanes<32>(acc[g][i].w);
      }
    const int w = tid >> 6, ln = tid & 63;
    if (w > 0 && ln < 32)
#pragma unroll
      for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int i = 0; i < ND4; ++i) {
          const int cg = c4 + i * a.lpk;
          if (i < a.nd4 && cg * 4 < a.dim) store4(xred + (size_t(w - 1) * GB + g) * a.dim, cg * 4, a.dim, acc[g][i]);
        }
    __syncthreads();
    if (tid < 32)
#pragma unroll
      for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int i = 0; i < ND4; ++i) {
          const int cg = c4 + i * a.lpk;
          if (i < a.nd4 && cg * 4 < a.dim)
            for (int l = 0; l < 3; ++l) {
              const float4 o = load4(xred + (size_t(l) * GB + g) * a.dim, cg * 4, a.dim);
              acc[g][i].x += o.x;
              acc[g][i].y += o.y;
              acc[g][i].z += o.z;
              acc[g][i].w += o.w;
            }
        }
  } else if (a.kl > 1) {
    if (kk < a.kl)
#pragma unroll
      for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int i = 0; i < ND4; ++i) {
          const int cg = c4 + i * a.lpk;
          if (i < a.nd4 && cg * 4 < a.dim) store4(xred + (size_t(kk) * GB + g) * a.dim, cg * 4, a.dim, acc[g][i]);
        }
    __syncthreads();
    if (kk == 0)
#pragma unroll
      for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int i = 0; i < ND4; ++i) {
          const int cg = c4 + i * a.lpk;
          if (i < a.nd4 && cg * 4 < a.dim)
            for (int l = 1; l < a.kl; ++l) {
              const float4 o = load4(xred + (size_t(l) * GB + g) * a.dim, cg * 4, a.dim);
              acc[g][i].x += o.x;
              acc[g][i].y += o.y;
              acc[g][i].z += o.z;
              acc[g][i].w += o.w;
            }
        }
  }
  if (kk != 0) return;
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const size_t row_head = size_t(r) * a.heads + h0 + g;
#pragma unroll
    for (int i = 0; i < ND4; ++i) {
      const int cg = c4 + i * a.lpk;
      if (i < a.nd4 && cg * 4 < a.dim) {
        float4 o = acc[g][i];
        if (a.splits == 1) {
          const float l = l_run[g];
          o = make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
          store4(out + row_head * a.dim, cg * 4, a.dim, o);
        } else {
          store4(opart + (size_t(s) * a.rows * a.heads + row_head) * a.dim, cg * 4, a.dim, o);
        }
      }
    }
    if (a.splits > 1 && tid == 0) {
      float *ml = mlpart + (size_t(s) * a.rows * a.heads + row_head) * 2;
      ml[0] = m_run[g];
      ml[1] = l_run[g];
    }
  }
}

// ---------------------------------------------------------------------------
// The 64-key chunk at dim 128 (a split of a few thousand keys).  q, the
// chunk's K^T rows (128 x 256 B) and its V rows (64 x 512 B) are requested
// straight into LDS, in that order, by buffer loads that write LDS: no
// registers hold them, so the whole chunk is in flight at once.  Each wave
// then waits for its q and K pieces only; the scores and the softmax run
// while V is still arriving, and the wave waits for V before the values.
// The arithmetic is k_attn's for this shape, in the same order (4 channel
// parts of 32 per key summed in part order; per head one online-softmax step
// over the 64 keys with the same lane butterflies, here head g in wave g % 4
// instead of all heads in wave 0; 8 key lanes of 8 keys each in key order,
// then the lane shuffle and the LDS sum of the four waves), so the two
// kernels give the same bits.
constexpr int kDmaKeys = 64, kDmaDim = 128;
constexpr int attn_dma_qfloats(int gb) { return gb * kDmaDim < 256 ? 256 : gb * kDmaDim; }  // whole 1 KiB pieces
constexpr size_t attn_dma_lds(int gb) {
  return size_t(2 * kDmaKeys * kDmaDim + attn_dma_qfloats(gb) + gb * kDmaKeys + 4 * gb +
                (3 * gb * kDmaDim > 4 * gb * kDmaKeys ? 3 * gb * kDmaDim : 4 * gb * kDmaKeys)) * 4;
}
typedef __amdgpu_buffer_rsrc_t AttnRsrc;
__device__ __forceinline__ AttnRsrc attn_rsrc(const void *base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(uint32_t(min(bytes, size_t(0xFFFFFFFFu)))),
                                           0x00020000);
}
// 1 KiB (16 B per lane, in lane order) from global memory at voff + soff into
// LDS at `lds` (wave-uniform).  The compiler does not see the LDS write: the
// waits before the barriers order it.  M0 is set here before each load;
// nothing else in k_attn_dma uses M0 (gfx950's LDS instructions do not read
// it), which the kernel's assembly shows.
__device__ __forceinline__ void attn_dma(AttnRsrc r, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff),
               "s"(r), "s"(soff)
               : "memory");
}
// Wait until at most N of this wave's vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void attn_vmwait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Phase timestamps of k_attn_dma, built only into libqnn_hip_trace.so
// (-DQNN_PHASE_TRACE): thread 0 of the workgroup with linear index w stores
// the device's real-time counter (100 MHz) at phase k; nothing else changes.
#ifdef QNN_PHASE_TRACE
constexpr int kAttnPhaseWGs = 2048, kAttnPhases = 16;
__device__ unsigned long long g_attn_phase[kAttnPhaseWGs * kAttnPhases];
#define QNN_ATTN_PHASE(k)                                                                                         \
  do {                                                                                                            \
    const unsigned w_ = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);                           \
    if (threadIdx.x == 0 && w_ < unsigned(kAttnPhaseWGs))                                                         \
      g_attn_phase[w_ * kAttnPhases + (k)] = __builtin_amdgcn_s_memrealtime();                                    \
  } while (0)
#else
#define QNN_ATTN_PHASE(k) \
  do {                    \
  } while (0)
#endif

template <int GB>
__global__ __launch_bounds__(kAttnThreads) void k_attn_dma(const float *__restrict__ q, const float *__restrict__ cache,
                                                           float *__restrict__ out, float *__restrict__ opart,
                                                           float *__restrict__ mlpart, AttnArgs a) {
  extern __shared__ float lds[];
  constexpr int QF = attn_dma_qfloats(GB);
  float *kls = lds;                          // [128 channels][64 keys]
  float *vls = kls + kDmaDim * kDmaKeys;     // [64 keys][128 channels]
  float *qs = vls + kDmaKeys * kDmaDim;      // [GB][128] (QF floats)
  float *ps = qs + QF;                       // [GB][64]
  float *red = ps + GB * kDmaKeys;           // [4][GB] (keep, sum, max; the fourth keeps xred 16-byte aligned)
  float *xred = red + 4 * GB;                // score parts [4][GB][64], then value lanes [3][GB][128]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kh = blockIdx.x / a.gpk, h0 = kh * a.group + (blockIdx.x % a.gpk) * GB;
  const int r = blockIdx.y, s = blockIdx.z;
  int start, end;
  key_range(a, r, start, end);
  const int k0 = start + s * kDmaKeys, nkeys = min(end - k0, kDmaKeys);  // none past the row's last key
  const size_t width = size_t(a.kv_heads) * kDmaDim;
  const float *kt = cache + size_t(kh) * kDmaDim * a.cap;
  const float *vb = cache + size_t(a.cap) * width + size_t(kh) * a.cap * kDmaDim;
  const unsigned *mask = reinterpret_cast<const unsigned *>(cache + 2 * size_t(a.cap) * width) + size_t(r) * a.cap;

  QNN_ATTN_PHASE(0);
  // 1) q, then K^T, then V of the chunk into LDS.  Wave w: q piece w (if any;
  //    GB heads of 128 floats are GB / 2 pieces, a lone head half of one),
  //    channels 32w..32w+31 of K^T (8 pieces of 4 channels x 64 keys), keys
  //    16w..16w+15 of V (8 pieces of 2 keys x 128 channels).  Loads past q's
  //    heads or past this KV head's K^T or V region return 0; keys past the
  //    chunk's end are loaded but never used.
  constexpr int QP = QF / 256;  // q pieces
  const int nk = max(nkeys, 0);
  {
    const uint32_t base = uint32_t(reinterpret_cast<uintptr_t>(lds));
    if (wave < QP) {
      const AttnRsrc qr = attn_rsrc(q + (size_t(r) * a.heads + h0) * kDmaDim, size_t(GB) * kDmaDim * 4);
      attn_dma(qr, __builtin_amdgcn_readfirstlane(base + 65536u + uint32_t(wave) * 1024u),
               uint32_t(wave) * 1024u + uint32_t(lane) * 16u, 0u);
    }
    if (nk > 0) {
      const AttnRsrc kr = attn_rsrc(kt, size_t(kDmaDim) * a.cap * 4);
      const AttnRsrc vr = attn_rsrc(vb, size_t(a.cap) * kDmaDim * 4);
      const uint32_t kvoff = uint32_t((size_t(wave * 32 + lane / 16) * a.cap + k0 + (lane % 16) * 4) * 4);
      const uint32_t vvoff = uint32_t((size_t(k0 + wave * 16 + lane / 32) * kDmaDim + (lane % 32) * 4) * 4);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        attn_dma(kr, __builtin_amdgcn_readfirstlane(base + uint32_t(wave * 8 + i) * 1024u), kvoff,
                 uint32_t(i) * 16u * uint32_t(a.cap));
#pragma unroll
      for (int i = 0; i < 8; ++i)
        attn_dma(vr, __builtin_amdgcn_readfirstlane(base + 32768u + uint32_t(wave * 8 + i) * 1024u), vvoff,
                 uint32_t(i) * 1024u);
      attn_vmwait<8>();  // q and K landed (V may still be in flight)
    } else {
      attn_vmwait<0>();
    }
  }
  __syncthreads();
  QNN_ATTN_PHASE(1);

  const float mul = a.scale > 0.0f ? a.scale : 1.0f / sqrtf(float(kDmaDim));
  float m_run[GB], l_run[GB], keep[GB];
  float4 acc[GB];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
    acc[g] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int key_t = lane, part = wave;  // scores: key, 32-channel part
  const int kk = tid / 32, c4 = tid % 32;  // values: key lane, float4 channel group
  if (nk > 0) {
    // ---- scores: part `wave` of the channels for key `lane`
    bool valid = key_t < nk;
    if (valid && a.masked) valid = mask[k0 + key_t] != 0u;
    float sc[GB];
#pragma unroll
    for (int g = 0; g < GB; ++g) sc[g] = 0.0f;
    if (valid) {
      float kv[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) kv[u] = kls[(part * 32 + u) * kDmaKeys + key_t];
#pragma unroll
      for (int u = 0; u < 32; ++u)
#pragma unroll
        for (int g = 0; g < GB; ++g) sc[g] += qs[g * kDmaDim + part * 32 + u] * kv[u];
    }
#pragma unroll
    for (int g = 0; g < GB; ++g) xred[(part * GB + g) * kDmaKeys + key_t] = sc[g];
    __syncthreads();
    // ---- head g's online-softmax step in wave g % 4
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      if (g % 4 != wave) continue;
      float v = xred[g * kDmaKeys + key_t];
      for (int p = 1; p < 4; ++p) v += xred[(p * GB + g) * kDmaKeys + key_t];
      v *= mul;
      if (a.softcap > 0.0f) v = a.softcap * tanhf(fminf(fmaxf(v / a.softcap, -20.0f), 20.0f));
      float mx = valid ? v : -INFINITY;
      mx = dev::wave_max_xor(mx);
      const float m_new = fmaxf(m_run[g], mx);
      const float kp = m_new == -INFINITY ? 1.0f : expf(m_run[g] - m_new);
      const float p = (valid && m_new > -INFINITY) ? expf(v - m_new) : 0.0f;
      ps[g * kDmaKeys + key_t] = p;
      const float ls = dev::wave_sum_xor(p);
      if (key_t == 0) {
        red[g] = kp;
        red[GB + g] = l_run[g] * kp + ls;
        red[2 * GB + g] = m_new;
      }
    }
    QNN_ATTN_PHASE(2);
    attn_vmwait<0>();  // V landed
    __syncthreads();   // publishes ps, the running state and every wave's V pieces
    QNN_ATTN_PHASE(3);
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      keep[g] = red[g];
      l_run[g] = red[GB + g];
      m_run[g] = red[2 * GB + g];
      acc[g].x *= keep[g];
      acc[g].y *= keep[g];
      acc[g].z *= keep[g];
      acc[g].w *= keep[g];
    }
    // ---- values: key lane kk takes keys kk, kk + 8, ..., in key order
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int key = kk + u * 8;
      if (key < nk) {
        const float4 v = *reinterpret_cast<const float4 *>(vls + key * kDmaDim + c4 * 4);
#pragma unroll
        for (int g = 0; g < GB; ++g) {
          const float w = ps[g * kDmaKeys + key];
          acc[g].x += w * v.x;
          acc[g].y += w * v.y;
          acc[g].z += w * v.z;
          acc[g].w += w * v.w;
        }
      }
    }
    __syncthreads();  // xred is rewritten below
    QNN_ATTN_PHASE(4);
  }
  // ---- the 8 key lanes: two per wave meet by a lane exchange (lanes 0-31
  //      take lanes 32-63; the upper lanes' sums are not used), then the
  //      four waves in LDS
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    acc[g].x += dev::xor_lanes<32>(acc[g].x);
    acc[g].y += dev::xor_lanes<32>(acc[g].y);
    acc[g].z += dev::xor_lanes<32>(acc[g].z);
    acc[g].w += dev::xor_lanes<32>(acc[g].w);
  }
  if (wave > 0 && lane < 32)
#pragma unroll
    for (int g = 0; g < GB; ++g)
      *reinterpret_cast<float4 *>(xred + (size_t(wave - 1) * GB + g) * kDmaDim + c4 * 4) = acc[g];
  __syncthreads();
  QNN_ATTN_PHASE(5);
  if (tid >= 32) return;
#pragma unroll
  for (int g = 0; g < GB; ++g)
    for (int l = 0; l < 3; ++l) {
      const float4 o = *reinterpret_cast<const float4 *>(xred + (size_t(l) * GB + g) * kDmaDim + c4 * 4);
      acc[g].x += o.x;
      acc[g].y += o.y;
      acc[g].z += o.z;
      acc[g].w += o.w;
    }
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const size_t row_head = size_t(r) * a.heads + h0 + g;
    float4 o = acc[g];
    if (a.splits == 1) {
      const float l = l_run[g];
      o = make_float4(o.x / l, o.y / l, o.z / l, o.w / l);
      *reinterpret_cast<float4 *>(out + row_head * kDmaDim + c4 * 4) = o;
    } else {
      *reinterpret_cast<float4 *>(opart + (size_t(s) * a.rows * a.heads + row_head) * kDmaDim + c4 * 4) = o;
    }
    if (a.splits > 1 && tid == 0) {
      float *ml = mlpart + (size_t(s) * a.rows * a.heads + row_head) * 2;
      ml[0] = m_run[g];
      ml[1] = l_run[g];
    }
  }
  QNN_ATTN_PHASE(6);
}

// Merge the key chunks: out = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M).
// One workgroup per (row, head).  Thread t owns float4 channel group t % G
// (G = dim / 4 groups, dim % 4 == 0) and every (256 / G)-th chunk from t / G;
// it requests all of its chunks' outputs first (up to kMergeLoads float4 in
// flight), then the (max, sum) pairs; the head's maximum and denominator come
// from wave reductions, and the chunk groups meet in LDS in a fixed order.
// Other shapes (dim % 4 != 0, more chunks than fit the loads) take
// k_attn_merge_general.
constexpr int kMergeLoads = 8;
__global__ __launch_bounds__(256) void k_attn_merge(float *out, const float *opart, const float *mlpart, int splits,
                                                    int row_heads, int dim) {
  __shared__ float wsh[256];
  __shared__ float red[2][4];
  __shared__ float4 acc4[256];
  const int rh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int groups = dim / 4, sg = 256 / groups;  // chunk groups
  const int c = tid % groups, gi = tid / groups;
  float4 x[kMergeLoads];
  const float4 *ob = reinterpret_cast<const float4 *>(opart + size_t(rh) * dim) + c;
  const size_t stride4 = size_t(row_heads) * groups;
#pragma unroll
  for (int u = 0; u < kMergeLoads; ++u) {
    const int sidx = gi + u * sg;
    x[u] = (gi < sg && sidx < splits) ? ob[size_t(sidx) * stride4] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // (max, sum) of chunk tid (splits <= 256)
  float m = -INFINITY, l = 0.0f;
  if (tid < splits) {
    const float2 ml = *reinterpret_cast<const float2 *>(mlpart + (size_t(tid) * row_heads + rh) * 2);
    m = ml.x;
    l = ml.y;
  }
  float M = dev::wave_max_xor(m);
  if (lane == 0) red[0][wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float w = m > -INFINITY ? expf(m - M) : 0.0f;
  wsh[tid] = w;
  float L = dev::wave_sum_xor(l * w);
  if (lane == 0) red[1][wave] = L;
  __syncthreads();
  L = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int u = 0; u < kMergeLoads; ++u) {
    const int sidx = gi + u * sg;
    if (gi < sg && sidx < splits) {
      const float ww = wsh[sidx];
      v.x += x[u].x * ww;
      v.y += x[u].y * ww;
      v.z += x[u].z * ww;
      v.w += x[u].w * ww;
    }
  }
  acc4[tid] = v;
  __syncthreads();
  if (gi == 0) {
    for (int j = 1; j < sg; ++j) {
      const float4 o = acc4[j * groups + c];
      v.x += o.x;
      v.y += o.y;
      v.z += o.z;
      v.w += o.w;
    }
    reinterpret_cast<float4 *>(out + size_t(rh) * dim)[c] = make_float4(v.x / L, v.y / L, v.z / L, v.w / L);
  }
}

constexpr int kMergeMaxSplits = 4096;
// Any shape: one workgroup per (row, head) and 256 channels; `sg` split
// groups of threads share a channel and walk the chunks sixteen loads at a
// time.
__global__ __launch_bounds__(256) void k_attn_merge_general(float *out, const float *opart, const float *mlpart,
                                                            int splits, int row_heads, int dim, int dspan, int sg) {
  __shared__ float wsh[kMergeMaxSplits];
  __shared__ float red[256];
  const int rh = blockIdx.x, tid = threadIdx.x;
  float m = -INFINITY;
  for (int s = tid; s < splits; s += 256) m = fmaxf(m, mlpart[(size_t(s) * row_heads + rh) * 2]);
  red[tid] = m;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
    __syncthreads();
  }
  m = red[0];
  __syncthreads();
  float l = 0.0f;
  for (int s = tid; s < splits; s += 256) {
    const float *ml = mlpart + (size_t(s) * row_heads + rh) * 2;
    const float w = ml[0] > -INFINITY ? expf(ml[0] - m) : 0.0f;
    wsh[s] = w;
    l += ml[1] * w;
  }
  red[tid] = l;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (tid < st) red[tid] += red[tid + st];
    __syncthreads();
  }
  l = red[0];
  __syncthreads();
  const int g = tid / dspan, d = blockIdx.y * dspan + tid % dspan;
  float v = 0.0f;
  if (g < sg && d < dim) {
    const float *base = opart + size_t(rh) * dim + d;
    const size_t stride = size_t(row_heads) * dim;
    int s = g;
    for (; s + 15 * sg < splits; s += 16 * sg) {
      float x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = base[size_t(s + u * sg) * stride];
#pragma unroll
      for (int u = 0; u < 16; ++u) v += x[u] * wsh[s + u * sg];
    }
    for (; s < splits; s += sg) v += base[size_t(s) * stride] * wsh[s];
  }
  red[tid] = v;
  __syncthreads();
  if (g == 0 && d < dim) {
    for (int j = 1; j < sg; ++j) v += red[j * dspan + tid];
    out[size_t(rh) * dim + d] = v / l;
  }
}

// ---------------------------------------------------------------------------
// SampleToken (Context.Implementation.inc:1137-1187; tensor.comp:123-199).
//
// Tokens are ranked by a 64-bit key: the order-preserving bits of the score
// (after the repetition penalty; -0 taken as +0) above the inverted token id,
// so a larger key is a higher score or, on equal scores, a lower id -- the
// order of tensor.comp:135-136 and :169.  Key 0 is "no token" (excluded by a
// 0xffffffff seen flag, NaN, or past the vocabulary); keys at or below that of
// (-FLT_MAX, 0xffffffff) are never picked, as the reference's rank loop never
// picks them (its running best starts there).
//
// Level 0 reads the logits and seen flags; a workgroup takes the exact top-k
// of its 4096 tokens.  Each wave ranks its own 1024: a threshold found by
// bisection over ballot counts keeps only the tokens that can be in the
// wave's top-k (at least k half-lane maxima reach it), those are compacted,
// and k rounds of a DPP wave-wide maximum rank them; wave 0 then ranks the
// four waves' lists.  Levels above read the previous level's keys.  When a
// level's keys fit one workgroup (tiles * k <= 4096) the last workgroup to
// finish ranks them and draws the token (tensor.comp:177-197).
constexpr int kSampleThreads = 256;
constexpr int kSamplePerThread = 16;
constexpr int kSampleTile = kSampleThreads * kSamplePerThread;
constexpr unsigned kNoToken = 0xffffffffu;
constexpr float kLowest = -3.402823466e38f;

__device__ __forceinline__ uint32_t order_bits(float s) {
  const uint32_t u = __float_as_uint(s == 0.0f ? 0.0f : s);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ uint64_t rank_key(float s, unsigned id) {
  return isnan(s) ? 0ull : (uint64_t(order_bits(s)) << 32) | uint32_t(~id);
}
// The key of the reference's starting best (-FLT_MAX, 0xffffffff).
__device__ __forceinline__ uint64_t floor_key() { return uint64_t(order_bits(kLowest)) << 32; }

// Wave-wide maximum of an unsigned word (all 64 lanes active), uniform
// result: row_shr 1, 2, 4, 8 leave each row's maximum in its lane 15,
// row_bcast 15 and 31 carry it to lane 63.  Lanes without a source read 0,
// the identity of the maximum.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x111, 0xf, 0xf, true)));  // row_shr:1
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x112, 0xf, 0xf, true)));  // row_shr:2
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x114, 0xf, 0xf, true)));  // row_shr:4
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x118, 0xf, 0xf, true)));  // row_shr:8
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x142, 0xa, 0xf, false)));  // row_bcast:15
  x = max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), 0x143, 0xc, 0xf, false)));  // row_bcast:31
  return uint32_t(__builtin_amdgcn_readlane(int(x), 63));
}

// Wave-wide maximum of 64-bit keys: the high words first; the low words only
// among the lanes that hold the highest high word.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) {
  const uint32_t hi = uint32_t(v >> 32), lo = uint32_t(v);
  const uint32_t mh = wave_max_u32(hi);
  const uint64_t at = __ballot(hi == mh);
  uint32_t ml;
  if (__popcll(at) == 1)
    ml = uint32_t(__builtin_amdgcn_readlane(int(lo), __ffsll(static_cast<long long>(at)) - 1));
  else
    ml = wave_max_u32(hi == mh ? lo : 0u);
  return (uint64_t(mh) << 32) | ml;
}

// k rounds over J candidate keys per lane: each takes the wave-wide best key
// below the previous pick; keys at or below the floor are never picked.
template <int J>
__device__ __forceinline__ void rank_rounds(const uint64_t (&c)[J], int k, uint64_t *out) {
  const uint64_t floor = floor_key();
  uint64_t prev = ~0ull;
  for (int rank = 0; rank < k; ++rank) {
    uint64_t b = 0ull;
#pragma unroll
    for (int i = 0; i < J; ++i) {
      const uint64_t v = c[i] < prev ? c[i] : 0ull;
      b = v > b ? v : b;
    }
    uint64_t best = wave_max_key(b);
    if (best < floor) best = floor;
    if ((threadIdx.x & 63) == 0) out[rank] = best;
    prev = best;
  }
}

template <int J>
__device__ __forceinline__ void rank_from(const uint64_t *scratch, int count, int k, uint64_t *out) {
  const int lane = threadIdx.x & 63;
  uint64_t c[J];
#pragma unroll
  for (int i = 0; i < J; ++i) c[i] = i * 64 + lane < count ? scratch[i * 64 + lane] : 0ull;
  rank_rounds<J>(c, k, out);
}

__device__ __forceinline__ uint64_t shfl_xor_key(uint64_t v, int m) {
  const int lo = __shfl_xor(int(uint32_t(v)), m), hi = __shfl_xor(int(uint32_t(v >> 32)), m);
  return (uint64_t(uint32_t(hi)) << 32) | uint32_t(lo);
}

// Sorts the wave's 64*J keys (element j*64 + lane in c[j]) into descending
// order with a bitonic network, then writes ranks 0..k-1 (keys at or below the
// floor become the floor).
template <int J>
__device__ __forceinline__ void sort_from(const uint64_t *scratch, int count, int k, uint64_t *out) {
  const int lane = threadIdx.x & 63;
  uint64_t c[J];
#pragma unroll
  for (int j = 0; j < J; ++j) c[j] = j * 64 + lane < count ? scratch[j * 64 + lane] : 0ull;
#pragma unroll
  for (int size = 2; size <= 64 * J; size <<= 1) {
#pragma unroll
    for (int stride = size / 2; stride > 0; stride >>= 1) {
      if (stride >= 64) {
        const int rs = stride / 64;
#pragma unroll
        for (int j = 0; j < J; ++j)
          if ((j & rs) == 0) {
            const int e = j * 64 + lane;
            const bool desc = (e & size) == 0;
            const uint64_t a = c[j], b = c[j | rs];
            const uint64_t hi = a > b ? a : b, lo = a > b ? b : a;
            c[j] = desc ? hi : lo;
            c[j | rs] = desc ? lo : hi;
          }
      } else {
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const int e = j * 64 + lane;
          const uint64_t other = shfl_xor_key(c[j], stride);
          const bool desc = (e & size) == 0, first = (lane & stride) == 0;
          const uint64_t hi = c[j] > other ? c[j] : other, lo = c[j] > other ? other : c[j];
          c[j] = (first == desc) ? hi : lo;
        }
      }
    }
  }
  const uint64_t floor = floor_key();
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int e = j * 64 + lane;
    if (e < k) out[e] = c[j] > floor ? c[j] : floor;
  }
  if (lane == 0)
    for (int e = 64 * J; e < k; ++e) out[e] = floor;
}

// Ranked top-k (k <= 64) of the wave's keys, N per lane, into out[0..k)
// (unfilled ranks get floor_key()).  scratch: 64 * N keys of LDS.
template <int N>
__device__ __forceinline__ void wave_topk(const uint64_t (&key)[N], int k, uint64_t *scratch, uint64_t *out) {
  const int lane = threadIdx.x & 63;
  if (k <= 2) {  // a round or two of the wave-wide maximum beats filtering
    rank_rounds<N>(key, k, out);
    return;
  }
  // Threshold: the largest T with at least k half-lane maxima whose score
  // bits reach T; every key of the top-k has score bits >= T.
  uint32_t hm0 = 0, hm1 = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t h = uint32_t(key[i] >> 32);
    if (i < (N + 1) / 2) hm0 = max(hm0, h);
    else hm1 = max(hm1, h);
  }
  uint32_t t = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    const int n = __popcll(__ballot(hm0 >= c)) + (N > 1 ? __popcll(__ballot(hm1 >= c)) : 0);
    if (n >= k) t = c;
  }
  // Compact the keys that reach it.
  int count = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const bool keep = key[i] != 0ull && uint32_t(key[i] >> 32) >= t;
    const uint64_t mask = __ballot(keep);
    if (keep) scratch[count + __popcll(mask & ((1ull << lane) - 1ull))] = key[i];
    count += __popcll(mask);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Few survivors (the usual case): sort them.  Many (ties, flat logits):
  // k rounds of the wave-wide maximum.
  const int per_lane = (count + 63) / 64;
  if (per_lane <= 1)
    sort_from<1>(scratch, count, k, out);
  else if (per_lane <= 2)
    sort_from<2>(scratch, count, k, out);
  else if (per_lane <= 4 || N <= 4)
    sort_from<(N < 4 ? N : 4)>(scratch, count, k, out);
  else if (per_lane <= 8 || N <= 8)
    rank_from<(N < 8 ? N : 8)>(scratch, count, k, out);
  else
    rank_from<N>(scratch, count, k, out);
}

struct SampleArgs {
  int count, k, tiles, level0, merge;
  float temperature, top_p, penalty, uniform;
};

// The workgroup's ranked top-k of its 4096 keys (16 per lane) into top[0..k).
__device__ __forceinline__ void group_topk(const uint64_t (&key)[kSamplePerThread], int k, uint64_t *scratch,
                                           uint64_t (*lists)[64], uint64_t *top) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  wave_topk<kSamplePerThread>(key, k, scratch + wave * 64 * kSamplePerThread, lists[wave]);
  __syncthreads();
  if (wave == 0) {
    uint64_t c4[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) c4[w] = lane < k ? lists[w][lane] : 0ull;
    wave_topk<4>(c4, k, scratch, top);
  }
  __syncthreads();
}

__global__ __launch_bounds__(kSampleThreads) void k_sample(unsigned *dst, const float *logits, const unsigned *seen,
                                                           const uint64_t *in_keys, uint64_t *out_keys,
                                                           unsigned *counter, SampleArgs a) {
  __shared__ uint64_t scratch[4 * 64 * kSamplePerThread];
  __shared__ uint64_t lists[4][64];
  __shared__ uint64_t top[64];
  __shared__ float top_w[64];
  __shared__ unsigned ids[64];
  __shared__ unsigned last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, tile = blockIdx.x;
  uint64_t key[kSamplePerThread];
  // Wave w holds items [w*1024, (w+1)*1024) of the tile, lane-strided.
#pragma unroll
  for (int i = 0; i < kSamplePerThread; ++i) {
    const unsigned item = unsigned(tile) * kSampleTile + unsigned(wave) * 1024 + unsigned(i) * 64 + lane;
    key[i] = 0ull;
    if (item < unsigned(a.count)) {
      if (a.level0) {
        const unsigned flag = seen[item];
        float score = logits[item];
        if (flag != 0u) score = score < 0.0f ? score * a.penalty : score / a.penalty;
        key[i] = flag != kNoToken ? rank_key(score, item) : 0ull;
      } else {
        key[i] = __hip_atomic_load(&in_keys[item], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  group_topk(key, a.k, scratch, lists, top);
  if (tid < a.k) __hip_atomic_store(&out_keys[size_t(tile) * a.k + tid], top[tid], __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  if (!a.merge) return;
  // One ticket per workgroup once its keys are stored.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == unsigned(a.tiles - 1);
  __syncthreads();
  if (!last) return;

  // The last workgroup ranks every tile's keys (at most 4096).
  const int count = a.tiles * a.k;
#pragma unroll
  for (int i = 0; i < kSamplePerThread; ++i) {
    const int c = wave * 1024 + i * 64 + lane;
    key[i] = c < count ? __hip_atomic_load(&out_keys[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
  }
  group_topk(key, a.k, scratch, lists, top);
  if (tid == 0) {
#pragma clang fp contract(off)
    const uint64_t floor = floor_key();
    for (int j = 0; j < a.k; ++j) {
      const bool none = top[j] <= floor;
      top_w[j] = none ? kLowest : from_order_bits(uint32_t(top[j] >> 32));
      ids[j] = none ? kNoToken : ~uint32_t(top[j]);
    }
    unsigned selected = ids[0];
    if (a.temperature > 0.0f && a.k > 1) {
      float total = 0.0f;
      const float maximum = top_w[0];
      for (int j = 0; j < a.k; ++j) {
        top_w[j] = expf((top_w[j] - maximum) / a.temperature);
        total += top_w[j];
      }
      float retained = 0.0f;
      int n = 0;
      do {
        retained += top_w[n];
        ++n;
      } while (n < a.k && retained < a.top_p * total);
      const float target = a.uniform * retained;
      float accumulated = 0.0f;
      selected = ids[n - 1];
      for (int j = 0; j < n; ++j) {
        accumulated += top_w[j];
        if (target < accumulated) {
          selected = ids[j];
          break;
        }
      }
    }
    dst[0] = selected;
    dev::reset_counter(counter, 0);
  }
}

int grid_of(int64_t n, int block) { return int((n + block - 1) / block); }

}  // namespace

void decode_rope(float *dst, const float *src, int n, int heads, int dim, int position, float theta, hipStream_t s) {
  k_rope<<<grid_of(n, 256), 256, 0, s>>>(dst, src, n, heads, dim, position, theta);
}

void decode_cache_write(float *cache, const float *k, const float *v, int n, int kv_heads, int dim, int cap,
                        int position, hipStream_t s) {
  k_cache_write<<<grid_of(n, 256), 256, 0, s>>>(cache, k, v, n, kv_heads, dim, cap, position);
}

void decode_seen(float *flags, const float *ids, int n, int vocab, hipStream_t s) {
  k_seen<<<grid_of(n, 256), 256, 0, s>>>(reinterpret_cast<unsigned *>(flags), reinterpret_cast<const unsigned *>(ids),
                                         n, unsigned(vocab));
}

void decode_gather(float *dst, const float *ids, const void *w, int kind, const float *scales, int rows, int dim,
                   int vocab, hipStream_t s) {
  const int n = rows * dim;
  k_gather<<<grid_of(n, 256), 256, 0, s>>>(dst, reinterpret_cast<const unsigned *>(ids), w, kind, scales, n, dim,
                                           vocab);
}

void decode_scale(float *dst, const float *src, int n, float a, float b, hipStream_t s) {
  k_scale<<<grid_of(n, 256), 256, 0, s>>>(dst, src, n, a, b);
}

void decode_softcap(float *dst, const float *src, int n, float cap, hipStream_t s) {
  k_softcap<<<grid_of(n, 256), 256, 0, s>>>(dst, src, n, cap);
}

AttnPlan attn_plan(int rows, int heads, int kv_heads, int dim, int position, int window) {
  AttnPlan p;
  const int group = heads / kv_heads;
  p.gb = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
  const int wgs = kv_heads * (group / p.gb) * rows;
  const int last_end = position + rows;
  const int longest = window > 0 ? std::min(window, last_end) : last_end;
  // About two workgroups per CU, chunks of at least 64 keys (measured on
  // MI355X: 512 / 64 beat 256 / 128 and 128 / 256 at 4k and 32k keys).
  const int target = std::max(1, tuning().attn_wgs);
  const int min_chunk = std::max(64, tuning().attn_min_chunk) / 64 * 64;
  int splits = std::max(1, std::min((target + wgs - 1) / wgs, (longest + min_chunk - 1) / min_chunk));
  splits = std::min(splits, kMergeMaxSplits);
  p.chunk = ((longest + splits - 1) / splits + 63) / 64 * 64;
  p.splits = (longest + p.chunk - 1) / p.chunk;
  p.part_floats = p.splits > 1 ? size_t(p.splits) * rows * heads * (size_t(dim) + 2) : 0;
  return p;
}

void attn_launch(const float *q, const float *cache, float *out, float *ws, const AttnPlan &p, int rows, int cap,
                 int heads, int kv_heads, int dim, int position, int window, float softcap, float scale, int masked,
                 hipStream_t s) {
  AttnArgs a;
  a.rows = rows;
  a.cap = cap;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.dim = dim;
  a.position = position;
  a.window = window;
  a.masked = masked;
  a.softcap = softcap;
  a.scale = scale;
  a.group = heads / kv_heads;
  a.gpk = a.group / p.gb;
  a.splits = p.splits;
  a.chunk = p.chunk;
  a.sub = std::min(p.chunk, kAttnSub);
  a.parts = kAttnThreads / a.sub;
  const int groups4 = (dim + 3) / 4;
  a.lpk = std::min(groups4, kAttnThreads);
  a.kl = kAttnThreads / a.lpk;
  a.nd4 = (groups4 + a.lpk - 1) / a.lpk;
  float *opart = ws, *ml = ws ? ws + size_t(p.splits) * rows * heads * dim : nullptr;
  const size_t xred = std::max(size_t(a.parts > 1 ? a.parts : 0) * p.gb * a.sub,
                               size_t(a.kl > 1 ? a.kl : 0) * p.gb * dim);
  const size_t lds = (size_t(p.gb) * dim + size_t(p.gb) * kAttnSub + p.gb * 4 + xred) * 4;
  dim3 grid(kv_heads * a.gpk, rows, p.splits);
  // The LDS-stream kernel: dim 128, 64-key chunks, every chunk start a multiple
  // of 4 keys (16-byte K^T pieces), and a capacity of whole 16-byte rows.
  bool dma = tuning().attn_dma != 0 && dim == kDmaDim && p.chunk == kDmaKeys && cap % 4 == 0 && a.kl == 8 &&
             a.lpk == 32 && a.parts == 4;
  for (int r = 0; dma && r < rows; ++r) {
    const int e = position + r + 1;
    dma = (window > 0 && e > window ? e - window : 0) % 4 == 0;
  }
  if (dma) {
    static bool attr[9] = {};
    const size_t dl = attn_dma_lds(p.gb);
    auto go = [&](auto kern) {
      if (!attr[p.gb]) {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      int(dl)),
                  "attention LDS size");
        attr[p.gb] = true;
      }
      kern<<<grid, kAttnThreads, dl, s>>>(q, cache, out, opart, ml, a);
    };
    switch (p.gb) {
      case 8: go(k_attn_dma<8>); break;
      case 4: go(k_attn_dma<4>); break;
      case 2: go(k_attn_dma<2>); break;
      default: go(k_attn_dma<1>); break;
    }
  }
#define QNN_ATTN(G, N) k_attn<G, N><<<grid, kAttnThreads, lds, s>>>(q, cache, out, opart, ml, a)
  if (dma) {
  } else if (a.nd4 == 1) {
    switch (p.gb) {
      case 8: QNN_ATTN(8, 1); break;
      case 4: QNN_ATTN(4, 1); break;
      case 2: QNN_ATTN(2, 1); break;
      default: QNN_ATTN(1, 1); break;
    }
  } else {
    switch (p.gb) {
      case 8: QNN_ATTN(8, 2); break;
      case 4: QNN_ATTN(4, 2); break;
      case 2: QNN_ATTN(2, 2); break;
      default: QNN_ATTN(1, 2); break;
    }
  }
#undef QNN_ATTN
  if (p.splits > 1) {
    const int groups = dim / 4;
    if (dim % 4 == 0 && groups <= 256 && p.splits <= 256 && p.splits <= kMergeLoads * (256 / groups)) {
      k_attn_merge<<<rows * heads, 256, 0, s>>>(out, opart, ml, p.splits, rows * heads, dim);
    } else {
      const int dspan = dim >= 256 ? 256 : dim > 128 ? 256 : dim > 64 ? 128 : 64;
      const int sg = 256 / dspan;
      dim3 mg(rows * heads, (dim + dspan - 1) / dspan);
      k_attn_merge_general<<<mg, 256, 0, s>>>(out, opart, ml, p.splits, rows * heads, dim, dspan, sg);
    }
  }
}

int attn_phase_read(void *dst, size_t bytes) {
#ifdef QNN_PHASE_TRACE
  const size_t n = std::min(bytes, sizeof(g_attn_phase));
  if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_attn_phase), n, 0, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  static const unsigned long long zeros[kAttnPhaseWGs * kAttnPhases] = {};
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_attn_phase), zeros, sizeof(g_attn_phase), 0, hipMemcpyHostToDevice) != hipSuccess)
    return -1;
  return int(n / 8);
#else
  (void)dst;
  (void)bytes;
  return -2;
#endif
}

size_t sample_workspace_floats(int vocab, int k) {
  size_t total = 0;
  for (int count = vocab;;) {
    const int tiles = (count + kSampleTile - 1) / kSampleTile;
    total += 2 * size_t(tiles) * k;  // 64-bit keys
    if (size_t(tiles) * k <= size_t(kSampleTile)) break;
    count = tiles * k;
  }
  return total;
}

void sample_launch(float *dst, const float *logits, const float *seen, float *ws, unsigned *counter, int vocab, int k,
                   float temperature, float top_p, float penalty, float uniform, hipStream_t s) {
  const uint64_t *in_keys = nullptr;
  uint64_t *keys = reinterpret_cast<uint64_t *>(ws);
  int count = vocab, level0 = 1;
  for (;;) {
    const int tiles = (count + kSampleTile - 1) / kSampleTile;
    const int merge = size_t(tiles) * k <= size_t(kSampleTile) ? 1 : 0;
    SampleArgs a{count, k, tiles, level0, merge, temperature, top_p, penalty, uniform};
    k_sample<<<tiles, kSampleThreads, 0, s>>>(reinterpret_cast<unsigned *>(dst), logits,
                                              reinterpret_cast<const unsigned *>(seen), in_keys, keys, counter, a);
    if (merge) break;
    in_keys = keys;
    keys += size_t(tiles) * k;
    count = tiles * k;
    level0 = 0;
  }
}

}  // namespace qnn
