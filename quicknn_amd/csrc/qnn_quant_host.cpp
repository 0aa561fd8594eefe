// qnn_quant_host.cpp -- host-side weight preparation.
//
//  * qnn_quantize_int4: QuickNN's INT4 packer (QuantizeInt4,
//    src/core/QuickNN.Quantization.Int4.pas:35-144): per group of 32, scale =
//    max|v|/7, q = Round(v/scale) clamped to [-7,7] (half-to-even), one
//    least-squares refit scale = sum(v*q)/sum(q*q) in double, stored as fp32,
//    then nibbles q+8 from the refitted scale; tail elements store 8.
//  * qnn_gguf_quantize: block encoders for synthetic GGML weights.  The
//    reference ships no GGUF quantizer; these produce valid blocks of the
//    layouts its decoders read (src/io/QuickNN.GGUF.Quantization.pas:136-253).
#include <algorithm>
#include <atomic>
#include <cfenv>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/qnn_hip.h"
#include "qnn_iq_grids.h"

namespace {

float f32_from_bits(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
uint32_t bits_from_f32(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// binary32 -> binary16, round to nearest even.
uint16_t to_half(float f) {
  uint32_t x = bits_from_f32(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return uint16_t(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
  if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // rounds to >= 65520 -> inf
  if (ax < 0x38800000u) {                                   // subnormal half
    float a = f32_from_bits(ax);
    uint32_t m = uint32_t(std::nearbyint(a * 16777216.0f));  // a / 2^-24
    return uint16_t(sign | m);
  }
  uint32_t e = (ax >> 23) - 112;
  uint32_t man = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (man >> 13);
  uint32_t rest = man & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
  return uint16_t(sign | h);
}
float from_half(uint16_t h) {
  uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
  if (e == 0) return (sign ? -1.0f : 1.0f) * float(m) * 5.9604644775390625e-8f;
  if (e == 31) return f32_from_bits(sign | 0x7f800000u | (m << 13));
  return f32_from_bits(sign | ((e + 112) << 23) | (m << 13));
}
void put_half(uint8_t *p, float v) {
  uint16_t h = to_half(v);
  p[0] = uint8_t(h & 255);
  p[1] = uint8_t(h >> 8);
}
int clampi(long v, int lo, int hi) { return int(std::min<long>(std::max<long>(v, lo), hi)); }
int rnd(float v) { return int(std::nearbyint(v)); }

long long round_half_even(double v) { return (long long)std::nearbyint(v); }

int pack_int4_row(const float *f32, const uint16_t *bf16, uint8_t *dst, int row, int cols, int row_bytes) {
  float vals[32];
  for (int group = 0; group * 32 < cols; ++group) {
    const int base = group * 32, count = std::min(32, cols - base);
    float maximum = 0.0f;
    for (int j = 0; j < count; ++j) {
      const size_t i = size_t(row) * cols + base + j;
      vals[j] = bf16 ? f32_from_bits(uint32_t(bf16[i]) << 16) : f32[i];
      if (!std::isfinite(vals[j])) return -1;
      maximum = std::max(maximum, std::fabs(vals[j]));
    }
    float scale = float(double(maximum) / 7.0);
    if (maximum > 0 && scale == 0) scale = maximum;
    if (scale > 0) {
      double num = 0.0;
      int den = 0;
      for (int j = 0; j < count; ++j) {
        const int q = clampi(long(round_half_even(double(vals[j]) / double(scale))), -7, 7);
        num += double(vals[j]) * double(q);
        den += q * q;
      }
      if (den > 0) scale = float(num / double(den));
    }
    uint8_t *blk = dst + size_t(row) * row_bytes + size_t(group) * 20;
    std::memcpy(blk, &scale, 4);
    for (int wd = 0; wd < 4; ++wd) {
      uint32_t word = 0;
      for (int nb = 0; nb < 8; ++nb) {
        const int j = wd * 8 + nb;
        int q = 0;
        if (j < count && scale > 0) q = clampi(long(round_half_even(double(vals[j]) / double(scale))), -7, 7);
        word |= uint32_t(q + 8) << (4 * nb);
      }
      std::memcpy(blk + 4 + 4 * wd, &word, 4);
    }
  }
  return 0;
}

// ---------------------------------------------------------------- GGML encoders
void enc_q8_0(const float *x, uint8_t *b) {
  float amax = 0;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
  put_half(b, amax / 127.0f);
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  for (int i = 0; i < 32; ++i) b[2 + i] = uint8_t(int8_t(d > 0 ? clampi(rnd(x[i] / d), -127, 127) : 0));
}

void enc_q4_k(const float *x, uint8_t *b) {
  std::memset(b, 0, 144);
  float scale[8], mins[8];
  for (int j = 0; j < 8; ++j) {
    float lo = 0, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) { lo = std::min(lo, x[j * 32 + i]); hi = std::max(hi, x[j * 32 + i]); }
    scale[j] = (hi - lo) / 15.0f;
    mins[j] = -lo;
  }
  const float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(mins, mins + 8);
  put_half(b, ms / 63.0f);
  put_half(b + 2, mm / 63.0f);
  const float d = from_half(uint16_t(b[0] | (b[1] << 8))), dmin = from_half(uint16_t(b[2] | (b[3] << 8)));
  int sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0 ? clampi(rnd(scale[j] / d), 0, 63) : 0;
    m[j] = dmin > 0 ? clampi(rnd(mins[j] / dmin), 0, 63) : 0;
  }
  for (int j = 0; j < 4; ++j) {
    b[4 + j] = uint8_t((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    b[8 + j] = uint8_t((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    b[12 + j] = uint8_t((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
  for (int i = 0; i < 256; ++i) {
    const int j = i / 32;
    const float s = d * float(sc[j]), off = dmin * float(m[j]);
    const int q = s > 0 ? clampi(rnd((x[i] + off) / s), 0, 15) : 0;
    b[16 + (i / 64) * 32 + i % 32] |= uint8_t(q << ((j & 1) * 4));
  }
}

void enc_q6_k(const float *x, uint8_t *b) {
  std::memset(b, 0, 210);
  float scale[16], amax_all = 0;
  for (int j = 0; j < 16; ++j) {
    float a = 0;
    for (int i = 0; i < 16; ++i) a = std::max(a, std::fabs(x[j * 16 + i]));
    scale[j] = a / 31.0f;
    amax_all = std::max(amax_all, scale[j]);
  }
  put_half(b + 208, amax_all / 127.0f);
  const float d = from_half(uint16_t(b[208] | (b[209] << 8)));
  for (int j = 0; j < 16; ++j) {
    const int sc = d > 0 ? clampi(rnd(scale[j] / d), -128, 127) : 0;
    b[192 + j] = uint8_t(int8_t(sc));
  }
  for (int i = 0; i < 256; ++i) {
    const float s = d * float(int8_t(b[192 + i / 16]));
    const int q = (s != 0 ? clampi(rnd(x[i] / s), -32, 31) : 0) + 32;
    const int part = i / 128, quarter = (i % 128) / 32, lane = i % 32;
    b[part * 64 + (quarter & 1) * 32 + lane] |= uint8_t((q & 15) << ((quarter / 2) * 4));
    b[128 + part * 32 + lane] |= uint8_t(((q >> 4) & 3) << (quarter * 2));
  }
}

void enc_q3_k(const float *x, uint8_t *b) {
  std::memset(b, 0, 110);
  float scale[16], smax = 0;
  for (int j = 0; j < 16; ++j) {
    float a = 0;
    for (int i = 0; i < 16; ++i) a = std::max(a, std::fabs(x[j * 16 + i]));
    scale[j] = a / 4.0f;
    smax = std::max(smax, scale[j]);
  }
  put_half(b + 108, smax / 31.0f);
  const float d = from_half(uint16_t(b[108] | (b[109] << 8)));
  int sc6[16];
  for (int g = 0; g < 16; ++g) {
    sc6[g] = (d > 0 ? clampi(rnd(scale[g] / d), -32, 31) : 0) + 32;
    b[96 + g % 8] |= uint8_t((sc6[g] & 15) << ((g / 8) * 4));
    b[104 + g % 4] |= uint8_t(((sc6[g] >> 4) & 3) << ((g / 4) * 2));
  }
  for (int i = 0; i < 256; ++i) {
    const float s = d * float(sc6[i / 16] - 32);
    const int q = s != 0 ? clampi(rnd(x[i] / s), -4, 3) : 0;
    const int low = q < 0 ? q + 4 : q;
    b[32 + (i / 128) * 32 + i % 32] |= uint8_t(low << (((i % 128) / 32) * 2));
    if (q >= 0) b[i % 32] |= uint8_t(1 << (i / 32));
  }
}

void enc_q2_k(const float *x, uint8_t *b) {
  std::memset(b, 0, 84);
  float scale[16], mins[16];
  for (int j = 0; j < 16; ++j) {
    float lo = 0, hi = -INFINITY;
    for (int i = 0; i < 16; ++i) { lo = std::min(lo, x[j * 16 + i]); hi = std::max(hi, x[j * 16 + i]); }
    scale[j] = (hi - lo) / 3.0f;
    mins[j] = -lo;
  }
  put_half(b + 80, *std::max_element(scale, scale + 16) / 15.0f);
  put_half(b + 82, *std::max_element(mins, mins + 16) / 15.0f);
  const float d = from_half(uint16_t(b[80] | (b[81] << 8))), dmin = from_half(uint16_t(b[82] | (b[83] << 8)));
  for (int j = 0; j < 16; ++j) {
    const int sc = d > 0 ? clampi(rnd(scale[j] / d), 0, 15) : 0;
    const int m = dmin > 0 ? clampi(rnd(mins[j] / dmin), 0, 15) : 0;
    b[j] = uint8_t(sc | (m << 4));
  }
  for (int i = 0; i < 256; ++i) {
    const int j = i / 16;
    const float s = d * float(b[j] & 15), off = dmin * float(b[j] >> 4);
    const int q = s > 0 ? clampi(rnd((x[i] + off) / s), 0, 3) : 0;
    b[16 + (i / 128) * 32 + i % 32] |= uint8_t(q << (((i % 128) / 32) * 2));
  }
}

// Q5_K (176 B): Q4_K's d, dmin and 6-bit scales and mins, 5-bit quants: the
// low 4 bits at 48 + (i/64)*32 + i%32 (nibble by sub-block parity), the fifth
// bit of element i in byte 16 + i%32, bit i/32.
void enc_q5_k(const float *x, uint8_t *b) {
  std::memset(b, 0, 176);
  float scale[8], mins[8];
  for (int j = 0; j < 8; ++j) {
    float lo = 0, hi = -INFINITY;
    for (int i = 0; i < 32; ++i) { lo = std::min(lo, x[j * 32 + i]); hi = std::max(hi, x[j * 32 + i]); }
    scale[j] = (hi - lo) / 31.0f;
    mins[j] = -lo;
  }
  put_half(b, *std::max_element(scale, scale + 8) / 63.0f);
  put_half(b + 2, *std::max_element(mins, mins + 8) / 63.0f);
  const float d = from_half(uint16_t(b[0] | (b[1] << 8))), dmin = from_half(uint16_t(b[2] | (b[3] << 8)));
  int sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0 ? clampi(rnd(scale[j] / d), 0, 63) : 0;
    m[j] = dmin > 0 ? clampi(rnd(mins[j] / dmin), 0, 63) : 0;
  }
  for (int j = 0; j < 4; ++j) {
    b[4 + j] = uint8_t((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    b[8 + j] = uint8_t((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    b[12 + j] = uint8_t((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
  for (int i = 0; i < 256; ++i) {
    const int j = i / 32;
    const float s = d * float(sc[j]), off = dmin * float(m[j]);
    const int q = s > 0 ? clampi(rnd((x[i] + off) / s), 0, 31) : 0;
    b[48 + (i / 64) * 32 + i % 32] |= uint8_t((q & 15) << ((j & 1) * 4));
    b[16 + i % 32] |= uint8_t(((q >> 4) & 1) << j);
  }
}

// IQ4_NL / IQ4_XS codebook (src/io/QuickNN.GGUF.Quantization.pas:34).
const int kIQ4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
int iq4_nearest(float v) {  // index of the codebook value nearest v
  int best = 0;
  for (int q = 1; q < 16; ++q)
    if (std::fabs(float(kIQ4[q]) - v) < std::fabs(float(kIQ4[best]) - v)) best = q;
  return best;
}
// 32 values with scale d: element i's nibble in byte i % 16, high half for i >= 16.
void put_iq4_32(const float *x, float d, uint8_t *qs) {
  std::memset(qs, 0, 16);
  for (int i = 0; i < 32; ++i) {
    const int q = d != 0 ? iq4_nearest(x[i] / d) : 8;  // codebook[8] = 1: small, any is exact for d = 0
    qs[i % 16] |= uint8_t(q << ((i / 16) * 4));
  }
}
// The signed value of largest magnitude, so that it maps onto codebook[0] = -127.
float signed_amax(const float *x, int n) {
  float m = 0;
  for (int i = 0; i < n; ++i)
    if (std::fabs(x[i]) > std::fabs(m)) m = x[i];
  return m;
}

// IQ4_NL (18 B per 32): fp16 d, 16 bytes of codebook nibbles.
void enc_iq4_nl(const float *x, uint8_t *b) {
  put_half(b, signed_amax(x, 32) / -127.0f);
  put_iq4_32(x, from_half(uint16_t(b[0] | (b[1] << 8))), b + 2);
}

// Q2_0 (18 B per 64): fp16 d, then 2-bit q, four elements to a byte (element
// i at bits 2(i % 4) of byte 2 + i / 4); value d * (q - 1), q - 1 in -1..2.
// d maps the largest-magnitude element to 2 or to -1, whichever leaves the
// smaller squared error.
void enc_q2_0(const float *x, uint8_t *b) {
  std::memset(b, 0, 18);
  const float m = signed_amax(x, 64);
  float best_d = 0.0f, best_err = -1.0f;
  for (float cand : {m / 2.0f, -m}) {
    const float d = from_half(to_half(cand));
    float err = 0.0f;
    for (int i = 0; i < 64; ++i) {
      const int q = d != 0 ? clampi(rnd(x[i] / d), -1, 2) : 0;
      const float e = x[i] - d * float(q);
      err += e * e;
    }
    if (best_err < 0 || err < best_err) { best_err = err; best_d = cand; }
  }
  put_half(b, best_d);
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  for (int i = 0; i < 64; ++i) {
    const int q = (d != 0 ? clampi(rnd(x[i] / d), -1, 2) : 0) + 1;
    b[2 + i / 4] |= uint8_t(q << ((i % 4) * 2));
  }
}

// ---- IQ2 / IQ3 grid formats.  Each 8 (IQ2) or 4 (IQ3) magnitudes |x| / delta
// take the nearest codebook entry (least squares, brute force), the signs
// are stored as bits.  IQ2_XXS and IQ3_XXS store 7 of 8 sign bits, the eighth
// being their parity: where the signs of 8 elements have odd parity, the
// element of least magnitude takes the other sign.
static constexpr auto kHostG2XXS = qnn_iq::iq2xxs_grid();
static constexpr auto kHostG2S = qnn_iq::iq2s_grid();
static constexpr auto kHostG3XXS = qnn_iq::iq3xxs_grid();
static constexpr auto kHostG3S = qnn_iq::iq3s_grid();

template <class T, int N>
int nearest_entry(const qnn_iq::Table<T, N> &grid, int bytes, const float *mag) {
  int best = 0;
  float best_err = INFINITY;
  for (int e = 0; e < N; ++e) {
    float err = 0.0f;
    for (int i = 0; i < bytes; ++i) {
      const float d = mag[i] - float((grid.v[e] >> (8 * i)) & 255u);
      err += d * d;
    }
    if (err < best_err) { best_err = err; best = e; }
  }
  return best;
}

// Sign bits of 8 elements (bit i: x[i] < 0); with `even`, forced to even parity.
uint32_t sign_bits8(const float *x, bool even) {
  uint32_t s = 0;
  int least = 0;
  for (int i = 0; i < 8; ++i) {
    if (x[i] < 0) s |= 1u << i;
    if (std::fabs(x[i]) < std::fabs(x[least])) least = i;
  }
  if (even && (__builtin_popcount(s) & 1)) s ^= 1u << least;
  return s;
}

float amax_of(const float *x, int n) {
  float m = 0;
  for (int i = 0; i < n; ++i) m = std::max(m, std::fabs(x[i]));
  return m;
}

// d for per-group steps delta_g = d * f(n_g), n_g in 0..15 with f(15) the largest step.
float grid_d(const float *x, int group, float top_level, float f15) {
  float m = 0;
  for (int g = 0; g < 256 / group; ++g) m = std::max(m, amax_of(x + g * group, group) / top_level);
  return m / f15;
}
int step_index(float want, float d, float unit, float offset) {  // n with d * (offset + n) * unit nearest want
  return d > 0 ? clampi(rnd(want / (d * unit) - offset), 0, 15) : 0;
}

// IQ2_XXS (66 B per 256): fp16 d; per 32-group 4 grid-index bytes and a word of
// 4 x 7 sign bits with a 4-bit scale n on top; delta = d (0.5 + n) / 4.
void enc_iq2_xxs(const float *x, uint8_t *b) {
  std::memset(b, 0, 66);
  put_half(b, grid_d(x, 32, 43.0f, 15.5f * 0.25f));
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  for (int g = 0; g < 8; ++g) {
    const float *xg = x + 32 * g;
    const int n = step_index(amax_of(xg, 32) / 43.0f, d, 0.25f, 0.5f);
    const float delta = d * (0.5f + float(n)) * 0.25f;
    uint32_t bits = uint32_t(n) << 28;
    for (int L = 0; L < 4; ++L) {
      float mag[8];
      for (int i = 0; i < 8; ++i) mag[i] = delta > 0 ? std::fabs(xg[8 * L + i]) / delta : 0.0f;
      b[2 + 8 * g + L] = uint8_t(nearest_entry(kHostG2XXS, 8, mag));
      bits |= (sign_bits8(xg + 8 * L, true) & 127u) << (7 * L);
    }
    std::memcpy(b + 6 + 8 * g, &bits, 4);
  }
}

// IQ2_S (82 B per 256): fp16 d, 32 low index bytes, 32 sign bytes, 8 bytes of
// 4 x 2 high index bits, 8 bytes of two 4-bit scales (per 16 elements).
void enc_iq2_s(const float *x, uint8_t *b) {
  std::memset(b, 0, 82);
  put_half(b, grid_d(x, 16, 43.0f, 15.5f * 0.25f));
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  for (int g = 0; g < 8; ++g) {
    for (int h = 0; h < 2; ++h) {
      const float *xh = x + 32 * g + 16 * h;
      const int n = step_index(amax_of(xh, 16) / 43.0f, d, 0.25f, 0.5f);
      const float delta = d * (0.5f + float(n)) * 0.25f;
      b[74 + g] |= uint8_t(n << (4 * h));
      for (int L = 2 * h; L < 2 * h + 2; ++L) {
        float mag[8];
        for (int i = 0; i < 8; ++i) mag[i] = delta > 0 ? std::fabs(x[32 * g + 8 * L + i]) / delta : 0.0f;
        const int e = nearest_entry(kHostG2S, 8, mag);
        b[2 + 4 * g + L] = uint8_t(e & 255);
        b[66 + g] |= uint8_t((e >> 8) << (2 * L));
        b[34 + 4 * g + L] = uint8_t(sign_bits8(x + 32 * g + 8 * L, false));
      }
    }
  }
}

// IQ3_XXS (98 B per 256): fp16 d, 64 grid-index bytes (one per 4 elements), 8
// words of 4 x 7 sign bits with a 4-bit scale n on top; delta = d (0.5 + n) / 2.
void enc_iq3_xxs(const float *x, uint8_t *b) {
  std::memset(b, 0, 98);
  put_half(b, grid_d(x, 32, 62.0f, 15.5f * 0.5f));
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  for (int g = 0; g < 8; ++g) {
    const float *xg = x + 32 * g;
    const int n = step_index(amax_of(xg, 32) / 62.0f, d, 0.5f, 0.5f);
    const float delta = d * (0.5f + float(n)) * 0.5f;
    uint32_t bits = uint32_t(n) << 28;
    for (int j = 0; j < 8; ++j) {
      float mag[4];
      for (int i = 0; i < 4; ++i) mag[i] = delta > 0 ? std::fabs(xg[4 * j + i]) / delta : 0.0f;
      b[2 + 8 * g + j] = uint8_t(nearest_entry(kHostG3XXS, 4, mag));
    }
    for (int L = 0; L < 4; ++L) bits |= (sign_bits8(xg + 8 * L, true) & 127u) << (7 * L);
    std::memcpy(b + 66 + 4 * g, &bits, 4);
  }
}

// IQ3_S (110 B per 256): fp16 d, 64 low index bytes, 8 bytes of high index
// bits, 32 sign bytes, 4 bytes of 4-bit scales s; step d (1 + 2 s).
void enc_iq3_s(const float *x, uint8_t *b) {
  std::memset(b, 0, 110);
  put_half(b, grid_d(x, 32, 15.0f, 31.0f));
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  for (int g = 0; g < 8; ++g) {
    const float *xg = x + 32 * g;
    const int s = d > 0 ? clampi(rnd((amax_of(xg, 32) / 15.0f / d - 1.0f) / 2.0f), 0, 15) : 0;
    const float step = d * float(1 + 2 * s);
    b[106 + g / 2] |= uint8_t(s << (4 * (g % 2)));
    for (int j = 0; j < 8; ++j) {
      float mag[4];
      for (int i = 0; i < 4; ++i) mag[i] = step > 0 ? std::fabs(xg[4 * j + i]) / step : 0.0f;
      const int e = nearest_entry(kHostG3S, 4, mag);
      b[2 + 8 * g + j] = uint8_t(e & 255);
      b[66 + g] |= uint8_t((e >> 8) << j);
    }
    for (int L = 0; L < 4; ++L) b[74 + 4 * g + L] = uint8_t(sign_bits8(xg + 8 * L, false));
  }
}

// IQ4_XS (136 B per 256): fp16 d, 6-bit signed sub-block scales (low nibbles
// at 4 + j/2, high 2 bits of scale j at bits 2j of the 16-bit word at 2),
// then 8 x 16 bytes of codebook nibbles.
void enc_iq4_xs(const float *x, uint8_t *b) {
  std::memset(b, 0, 136);
  float s[8], smax = 0;
  for (int j = 0; j < 8; ++j) {
    s[j] = signed_amax(x + 32 * j, 32) / -127.0f;
    if (std::fabs(s[j]) > std::fabs(smax)) smax = s[j];
  }
  put_half(b, smax / -32.0f);
  const float d = from_half(uint16_t(b[0] | (b[1] << 8)));
  uint32_t high = 0;
  for (int j = 0; j < 8; ++j) {
    const int ls = (d != 0 ? clampi(rnd(s[j] / d), -32, 31) : 0) + 32;
    b[4 + j / 2] |= uint8_t((ls & 15) << ((j % 2) * 4));
    high |= uint32_t((ls >> 4) & 3) << (2 * j);
    put_iq4_32(x + 32 * j, d * float(ls - 32), b + 8 + 16 * j);
  }
  b[2] = uint8_t(high & 255);
  b[3] = uint8_t(high >> 8);
}

}  // namespace

extern "C" {

int qnn_int4_row_bytes(int cols) {
  if (cols < 1) return -1;
  const long long bytes = ((long long)cols + 31) / 32 * 20;
  return bytes > 0x7fffffffLL ? -1 : int(bytes);
}

int qnn_quantize_int4(const void *src, int dtype, int rows, int cols, uint8_t *dst) {
  if (!src || !dst || rows < 1 || cols < 1 || (dtype != QNN_DT_F32 && dtype != QNN_DT_BF16)) return QNN_E_ARGUMENT;
  const int rb = qnn_int4_row_bytes(cols);
  if (rb < 0) return QNN_E_ARGUMENT;
  std::fesetround(FE_TONEAREST);
  const float *f32 = dtype == QNN_DT_F32 ? static_cast<const float *>(src) : nullptr;
  const uint16_t *b16 = dtype == QNN_DT_BF16 ? static_cast<const uint16_t *>(src) : nullptr;
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int threads = (rows >= 64 && (long long)rows * cols >= 32768) ? int(std::min(hw, 64u)) : 1;
  std::atomic<int> bad{0};
  auto work = [&](int t) {
    for (long long r = (long long)rows * t / threads; r < (long long)rows * (t + 1) / threads; ++r)
      if (pack_int4_row(f32, b16, dst, int(r), cols, rb)) bad = 1;
  };
  if (threads == 1) {
    work(0);
  } else {
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t) ts.emplace_back(work, t);
    for (auto &t : ts) t.join();
  }
  return bad ? QNN_E_ARGUMENT : QNN_OK;
}

int qnn_gguf_quantize(int encoding, const float *src, int64_t n, uint8_t *dst) {
  int elems, bytes;
  void (*fn)(const float *, uint8_t *);
  switch (encoding) {
    case QNN_WE_Q8_0: elems = 32; bytes = 34; fn = enc_q8_0; break;
    case QNN_WE_Q4_K: elems = 256; bytes = 144; fn = enc_q4_k; break;
    case QNN_WE_Q6_K: elems = 256; bytes = 210; fn = enc_q6_k; break;
    case QNN_WE_Q3_K: elems = 256; bytes = 110; fn = enc_q3_k; break;
    case QNN_WE_Q2_K: elems = 256; bytes = 84; fn = enc_q2_k; break;
    case QNN_WE_Q5_K: elems = 256; bytes = 176; fn = enc_q5_k; break;
    case QNN_WE_IQ4_NL: elems = 32; bytes = 18; fn = enc_iq4_nl; break;
    case QNN_WE_IQ4_XS: elems = 256; bytes = 136; fn = enc_iq4_xs; break;
    case QNN_WE_Q2_0: elems = 64; bytes = 18; fn = enc_q2_0; break;
    case QNN_WE_IQ2_XXS: elems = 256; bytes = 66; fn = enc_iq2_xxs; break;
    case QNN_WE_IQ2_S: elems = 256; bytes = 82; fn = enc_iq2_s; break;
    case QNN_WE_IQ3_XXS: elems = 256; bytes = 98; fn = enc_iq3_xxs; break;
    case QNN_WE_IQ3_S: elems = 256; bytes = 110; fn = enc_iq3_s; break;
    default: return QNN_E_NOT_SUPPORTED;
  }
  if (!src || !dst || n < 0 || n % elems) return QNN_E_ARGUMENT;
  const int64_t nb = n / elems;
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int threads = nb >= 4096 ? int(std::min(hw, 64u)) : 1;
  std::atomic<int> bad{0};
  auto work = [&](int t) {
    for (int64_t blk = nb * t / threads; blk < nb * (t + 1) / threads; ++blk) {
      const float *x = src + blk * elems;
      for (int i = 0; i < elems; ++i)
        if (!std::isfinite(x[i])) bad = 1;
      fn(x, dst + blk * bytes);
    }
  };
  if (threads == 1) {
    work(0);
  } else {
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t) ts.emplace_back(work, t);
    for (auto &t : ts) t.join();
  }
  return bad ? QNN_E_ARGUMENT : QNN_OK;
}

}  // extern "C"
