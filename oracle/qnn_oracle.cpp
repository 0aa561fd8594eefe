// qnn_oracle.cpp -- CPU restatement of QuickNN's quantized-decode path.
//
// TEST INFRASTRUCTURE ONLY: this is the checker for the HIP backend and the
// CPU baseline timed beside it.  It is never linked into the product library.
// Built with: g++ -O2 -mavx2 -mf16c -ffp-contract=off (no FMA contraction), so
// that every multiply and add rounds separately, as in the reference's AVX2
// assembly (vmulps / vaddps pairs).
//
// Reference paths are relative to the QuickNN source tree.
#include "qnn_oracle.h"
// The IQ2/IQ3 codebooks (GGML's; the reference's src/io/QuickNN.GGUF.Tables.inc),
// pinned against digests of the reference's tables in tests/test_oracle_gguf.py.
#include "../quicknn_amd/csrc/qnn_iq_grids.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cfenv>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

inline float bits_to_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t float_to_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// Exact binary16 -> binary32 conversion (the reference uses a table method,
// src/core/QuickNN.Common.pas:1799+, and vcvtph2ps in asm; both are exact).
inline float half_to_float(uint16_t h) {
  uint32_t sign = uint32_t(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do { man <<= 1; ++e; } while (!(man & 0x400));
      man &= 0x3ff;
      out = sign | (uint32_t(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    out = sign | 0x7f800000u | (man << 13);
  } else {
    out = sign | ((exp + 112) << 23) | (man << 13);
  }
  return bits_to_float(out);
}

inline float half_at(const uint8_t *p) { return half_to_float(uint16_t(p[0] | (p[1] << 8))); }
inline int signed_byte(uint8_t v) { return v >= 128 ? int(v) - 256 : int(v); }

// ---------------------------------------------------------------------------
// Horizontal reduction shared by every AVX2 dot in the reference:
//   vextractf128 xmm1, ymm0, 1 ; vaddps xmm0, xmm0, xmm1 ; vhaddps ; vhaddps
// (e.g. src/backends/cpu/QuickNN.CPU.Inference.AVX2.inc:51-54).
inline float hreduce(__m256 acc) {
  __m128 lo = _mm256_castps256_ps128(acc);
  __m128 hi = _mm256_extractf128_ps(acc, 1);
  __m128 s = _mm_add_ps(lo, hi);
  s = _mm_hadd_ps(s, s);
  s = _mm_hadd_ps(s, s);
  return _mm_cvtss_f32(s);
}

inline __m256 load_u8x8_epi32_ps(const uint8_t *p) {  // vpmovzxbd ymm, qword [p] ; vcvtdq2ps
  __m128i v = _mm_loadl_epi64(reinterpret_cast<const __m128i *>(p));
  return _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(v));
}
inline __m256i load_u8x8_epi32(const uint8_t *p) {
  __m128i v = _mm_loadl_epi64(reinterpret_cast<const __m128i *>(p));
  return _mm256_cvtepu8_epi32(v);
}

// ---------------------------------------------------------------------------
// Thread pool: TInferencePool (src/backends/cpu/QuickNN.CPU.Inference.pas:109-158).
// Persistent workers; the caller runs job(0); Run is not re-entrant.
struct Pool {
  int threads = 1;
  std::vector<std::thread> workers;
  std::mutex mu;
  std::condition_variable cv_start, cv_done;
  std::function<void(int)> job;
  uint64_t generation = 0;
  int pending = 0;
  bool stop = false;

  explicit Pool(int t) : threads(t) {
    for (int i = 1; i < threads; ++i) workers.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu);
      stop = true;
    }
    cv_start.notify_all();
    for (auto &w : workers) w.join();
  }
  void loop(int index) {
    uint64_t seen = 0;
    for (;;) {
      std::function<void(int)> j;
      {
        std::unique_lock<std::mutex> g(mu);
        cv_start.wait(g, [&] { return stop || generation != seen; });
        if (stop) return;
        seen = generation;
        j = job;
      }
      j(index);
      {
        std::lock_guard<std::mutex> g(mu);
        if (--pending == 0) cv_done.notify_all();
      }
    }
  }
  void run(const std::function<void(int)> &f) {
    if (threads == 1) { f(0); return; }
    {
      std::lock_guard<std::mutex> g(mu);
      job = f;
      pending = threads - 1;
      ++generation;
    }
    cv_start.notify_all();
    f(0);
    std::unique_lock<std::mutex> g(mu);
    cv_done.wait(g, [&] { return pending == 0; });
  }
};

// Round(Double) in Delphi: round-half-to-even under the default rounding mode.
inline long long delphi_round(double v) { return (long long)std::nearbyint(v); }
inline int ensure_range(long long v, int lo, int hi) { return int(std::min<long long>(std::max<long long>(v, lo), hi)); }

}  // namespace

extern "C" {

float qo_half_to_float(uint16_t h) { return half_to_float(h); }

uint16_t qo_float_to_half(float f) {
  __m128 v = _mm_set_ss(f);
  __m128i h = _mm_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  return uint16_t(_mm_extract_epi16(h, 0));
}

// ===========================================================================
// INT4: src/core/QuickNN.Quantization.Int4.pas
// ===========================================================================
int qo_int4_row_bytes(int cols) {  // :25-33
  if (cols < 1) return -1;
  long long bytes = ((long long)cols + 31) / 32 * 20;
  if (bytes > 0x7fffffffLL) return -1;
  return int(bytes);
}

// PackInt4Row (:35-94).  Max-abs/7 scale, round half-even to [-7,7],
// least-squares refit in double, store fp32 scale + offset-binary nibbles.
static int pack_int4_row(const float *f32, const uint16_t *bf16, uint8_t *dst, int row, int cols, int row_bytes) {
  float values[32];
  for (int group = 0; group <= (cols - 1) / 32; ++group) {
    int base = group * 32;
    int count = std::min(32, cols - base);
    float maximum = 0;
    for (int j = 0; j < count; ++j) {
      size_t idx = size_t(row) * cols + base + j;
      values[j] = bf16 ? bits_to_float(uint32_t(bf16[idx]) << 16) : f32[idx];
      if (!std::isfinite(values[j])) return -1;  // EArgumentException (:58-59)
      maximum = std::max(maximum, std::fabs(values[j]));
    }
    float scale = float(double(maximum) / 7.0);  // :62 (Single / Integer)
    if (maximum > 0 && scale == 0) scale = maximum;  // :63-64
    if (scale > 0) {  // :65-77
      double numerator = 0;
      int denominator = 0;
      for (int j = 0; j < count; ++j) {
        int q = ensure_range(delphi_round(double(values[j]) / double(scale)), -7, 7);
        numerator = numerator + double(values[j]) * double(q);
        denominator += q * q;
      }
      if (denominator > 0) scale = float(numerator / double(denominator));
    }
    uint8_t *block = dst + size_t(row) * row_bytes + size_t(group) * 20;  // :78-92
    std::memcpy(block, &scale, 4);
    for (int w = 0; w < 4; ++w) {
      uint32_t word = 0;
      for (int n = 0; n < 8; ++n) {
        int j = w * 8 + n;
        int q = 0;
        if (j < count && scale > 0) q = ensure_range(delphi_round(double(values[j]) / double(scale)), -7, 7);
        word |= uint32_t(q + 8) << (n * 4);
      }
      std::memcpy(block + 4 + w * 4, &word, 4);
    }
  }
  return 0;
}

int qo_quantize_int4(const void *src, int is_bf16, int rows, int cols, uint8_t *dst) {  // :96-144
  if (!src || !dst || rows < 1 || cols < 1) return -1;
  int row_bytes = qo_int4_row_bytes(cols);
  if (row_bytes < 0) return -1;
  std::fesetround(FE_TONEAREST);
  const float *f32 = is_bf16 ? nullptr : static_cast<const float *>(src);
  const uint16_t *b16 = is_bf16 ? static_cast<const uint16_t *>(src) : nullptr;
  // The reference parallelises over rows (TParallel.For, :128-135); rows are
  // independent so the result does not depend on the split.
  int threads = (rows >= 64 && (long long)rows * cols >= 32768) ? int(std::min(8u, std::max(1u, std::thread::hardware_concurrency()))) : 1;
  std::atomic<int> status{0};
  auto work = [&](int t) {
    for (int r = (long long)rows * t / threads; r < (long long)rows * (t + 1) / threads; ++r)
      if (pack_int4_row(f32, b16, dst, r, cols, row_bytes) != 0) status = -1;
  };
  if (threads == 1) work(0);
  else {
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t) ts.emplace_back(work, t);
    for (auto &t : ts) t.join();
  }
  return status.load();
}

// Scalar dequant (src/backends/cpu/QuickNN.CPU.Inference.pas:413-420): one
// rounding of the exact product (n-8)*s.
float qo_int4_value(const uint8_t *row, int k) {
  const uint8_t *base = row + (k / 32) * 20;
  int j = k % 32;
  float s;
  std::memcpy(&s, base, 4);
  int n = (base[4 + j / 2] >> ((j & 1) * 4)) & 15;
  return float(n - 8) * s;
}

void qo_int4_dequant_row(const uint8_t *row, int cols, float *out) {
  for (int k = 0; k < cols; ++k) out[k] = qo_int4_value(row, k);
}

// ===========================================================================
// GGUF formats: src/io/QuickNN.GGUF.Quantization.pas
// ===========================================================================
int qo_gguf_block_elements(int enc) {  // :67-75
  switch (enc) {
    case QO_ENC_Q8_0: case QO_ENC_IQ4_NL: return 32;
    case QO_ENC_Q2_0: return 64;
    case QO_ENC_IQ2_XXS: case QO_ENC_IQ2_S: case QO_ENC_IQ3_XXS: case QO_ENC_IQ3_S: return 256;
    case QO_ENC_Q4_K: case QO_ENC_Q6_K: case QO_ENC_Q3_K: case QO_ENC_Q2_K: case QO_ENC_Q5_K: case QO_ENC_IQ4_XS:
      return 256;
    default: return -1;
  }
}
int qo_gguf_block_bytes(int enc) {  // :77-93
  switch (enc) {
    case QO_ENC_Q8_0: return 34;
    case QO_ENC_Q2_K: return 84;
    case QO_ENC_Q4_K: return 144;
    case QO_ENC_Q6_K: return 210;
    case QO_ENC_Q3_K: return 110;
    case QO_ENC_Q5_K: return 176;
    case QO_ENC_IQ4_NL: return 18;
    case QO_ENC_IQ4_XS: return 136;
    case QO_ENC_Q2_0: return 18;
    case QO_ENC_IQ2_XXS: return 66;
    case QO_ENC_IQ2_S: return 82;
    case QO_ENC_IQ3_XXS: return 98;
    case QO_ENC_IQ3_S: return 110;
    default: return -1;
  }
}

// IQ2_XXS_GRID, IQ2_S_GRID, IQ3_XXS_GRID, IQ3_S_GRID, IQ2_SIGNS (Tables.inc:20-309).
static constexpr auto kG2XXS = qnn_iq::iq2xxs_grid();
static constexpr auto kG2S = qnn_iq::iq2s_grid();
static constexpr auto kG3XXS = qnn_iq::iq3xxs_grid();
static constexpr auto kG3S = qnn_iq::iq3s_grid();
static constexpr auto kSigns = qnn_iq::iq2_signs();

int qo_iq_table(int which, uint8_t *out) {
  const void *p;
  int n;
  switch (which) {
    case 0: p = kG2XXS.v; n = sizeof(kG2XXS.v); break;
    case 1: p = kG2S.v; n = sizeof(kG2S.v); break;
    case 2: p = kG3XXS.v; n = sizeof(kG3XXS.v); break;
    case 3: p = kG3S.v; n = sizeof(kG3S.v); break;
    case 4: p = kSigns.v; n = sizeof(kSigns.v); break;
    default: return -1;
  }
  if (out) std::memcpy(out, p, size_t(n));
  return n;
}

static uint32_t le32(const uint8_t *p) { return p[0] | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24); }

// IQ4_NL_VALUES (:34): the non-linear 4-bit codebook of IQ4_NL and IQ4_XS.
static const int kIQ4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// GGUFValue (:136-253), the scalar per-element decode.
float qo_gguf_value(const uint8_t *data, int enc, int64_t index) {
  int block = qo_gguf_block_elements(enc);
  const uint8_t *b = data + (index / block) * qo_gguf_block_bytes(enc);
  int i = int(index % block);
  switch (enc) {
    case QO_ENC_Q8_0:  // :180-181
      return half_at(b) * float(signed_byte(b[2 + i]));
    case QO_ENC_Q2_K: {  // :182-188
      int group = i / 16;
      int q = (b[16 + (i / 128) * 32 + i % 32] >> (((i % 128) / 32) * 2)) & 3;
      return (half_at(b + 80) * float(b[group] & 15)) * float(q) - half_at(b + 82) * float(b[group] >> 4);
    }
    case QO_ENC_Q4_K:
    case QO_ENC_Q5_K: {  // :189-207 (Q5_K: quants at 48, the fifth bit from byte 16 + i % 32)
      int group = i / 32, scale, minimum;
      if (group < 4) {
        scale = b[4 + group] & 63;
        minimum = b[8 + group] & 63;
      } else {
        scale = (b[8 + group] & 15) | ((b[group] >> 6) << 4);
        minimum = (b[8 + group] >> 4) | ((b[4 + group] >> 6) << 4);
      }
      const int quant_offset = enc == QO_ENC_Q5_K ? 48 : 16;
      int q = (b[quant_offset + (i / 64) * 32 + i % 32] >> ((group & 1) * 4)) & 15;
      if (enc == QO_ENC_Q5_K) q |= ((b[16 + i % 32] >> group) & 1) << 4;
      return (half_at(b) * float(scale)) * float(q) - half_at(b + 2) * float(minimum);
    }
    case QO_ENC_IQ3_XXS: {  // :148-157 (Pascal evaluates the scale in double; every value here is exact)
      const int group = i / 32;
      const uint32_t bits = le32(b + 66 + group * 4);
      const uint32_t signs = kSigns.v[(bits >> (7 * ((i % 32) / 8))) & 127];
      int q = int((kG3XXS.v[b[2 + i / 4]] >> ((i % 4) * 8)) & 255);
      if (signs & (1u << (i % 8))) q = -q;
      return float((double(half_at(b)) * (0.5 + double(bits >> 28)) * 0.5) * q);
    }
    case QO_ENC_IQ2_XXS:
    case QO_ENC_IQ2_S: {  // :158-179
      const int group = i / 32, lane = (i % 32) / 8;
      uint64_t grid;
      uint32_t signs;
      float delta;
      if (enc == QO_ENC_IQ2_XXS) {
        const uint32_t quant_bits = le32(b + 6 + group * 8);
        grid = kG2XXS.v[b[2 + group * 8 + lane]];
        signs = kSigns.v[(quant_bits >> (7 * lane)) & 127];
        delta = float(double(half_at(b)) * (0.5 + double(quant_bits >> 28)) * 0.25);
      } else {
        grid = kG2S.v[b[2 + group * 4 + lane] | (((b[66 + group] >> (lane * 2)) & 3) << 8)];
        signs = b[34 + i / 8];
        const int q = (b[74 + group] >> (((i % 32) / 16) * 4)) & 15;
        delta = float(double(half_at(b)) * (0.5 + q) * 0.25);
      }
      int q = int((grid >> ((i % 8) * 8)) & 255);
      if (signs & (1u << (i % 8))) q = -q;
      return delta * float(q);
    }
    case QO_ENC_IQ3_S: {  // :242-251
      const int group = i / 32;
      const int grid_index = b[2 + i / 4] | (((b[66 + group] >> ((i % 32) / 4)) & 1) << 8);
      int q = int((kG3S.v[grid_index] >> ((i % 4) * 8)) & 255);
      if (b[74 + i / 8] & (1 << (i % 8))) q = -q;
      const int scale = 1 + 2 * ((b[106 + group / 2] >> ((group % 2) * 4)) & 15);
      return (half_at(b) * float(scale)) * float(q);
    }
    case QO_ENC_Q2_0:  // :146-147: fp16 d, then 2-bit q four to a byte; d * (q - 1)
      return half_at(b) * float(int((b[2 + i / 4] >> ((i % 4) * 2)) & 3) - 1);
    case QO_ENC_IQ4_NL: {  // :229-233
      int q = (b[2 + i % 16] >> ((i / 16) * 4)) & 15;
      return half_at(b) * float(kIQ4[q]);
    }
    case QO_ENC_IQ4_XS: {  // :234-241
      int group = i / 32;
      int scale = ((b[4 + group / 2] >> ((group % 2) * 4)) & 15) | ((((int(b[2]) | (int(b[3]) << 8)) >> (group * 2)) & 3) << 4);
      int q = (b[8 + group * 16 + i % 16] >> (((i % 32) / 16) * 4)) & 15;
      return (half_at(b) * float(scale - 32)) * float(kIQ4[q]);
    }
    case QO_ENC_Q6_K: {  // :208-219
      int part = i / 128, quarter = (i % 128) / 32, lane = i % 32;
      int low = part * 64 + (quarter & 1) * 32 + lane;
      int high = 128 + part * 32 + lane;
      int q = ((b[low] >> ((quarter / 2) * 4)) & 15) | (((b[high] >> (quarter * 2)) & 3) << 4);
      int scale = signed_byte(b[192 + i / 16]);
      return (half_at(b + 208) * float(scale)) * float(q - 32);
    }
    case QO_ENC_Q3_K: {  // :220-228
      int group = i / 16;
      int scale = ((b[96 + group % 8] >> ((group / 8) * 4)) & 15) | (((b[104 + group % 4] >> ((group / 4) * 2)) & 3) << 4);
      int q = (b[32 + (i / 128) * 32 + i % 32] >> (((i % 128) / 32) * 2)) & 3;
      if ((b[i % 32] & (1 << (i / 32))) == 0) q -= 4;
      return (half_at(b + 108) * float(scale - 32)) * float(q);
    }
  }
  return std::nanf("");
}

// GGUFDecodeBlock AVX2 branch (:290-364) with DecodeLow4 / DecodeBits /
// DecodeSigned32 (src/io/QuickNN.GGUF.Decode.AVX2.inc:7-83): per-subblock
// Scale = d*sc and Bias = -(dmin*m), then cvt(q)*Scale + Bias.
// DecodeIQ4 (Decode.AVX2.inc:85-118): 16 bytes, low nibbles are elements
// 0-15 and high nibbles 16-31, each cvt(codebook byte) * scale.
static void decode_iq4(const uint8_t *src, float *dst, float scale) {
  for (int i = 0; i < 32; ++i) {
    const int q = (src[i % 16] >> ((i / 16) * 4)) & 15;
    dst[i] = float(kIQ4[q]) * scale;
  }
}

int qo_gguf_decode_block(const uint8_t *b, int enc, float *out) {
  switch (enc) {
    case QO_ENC_Q2_0:  // :285-289: element by element through GGUFValue
    case QO_ENC_IQ2_XXS:
    case QO_ENC_IQ2_S:
    case QO_ENC_IQ3_XXS:
      for (int i = 0; i < qo_gguf_block_elements(enc); ++i) out[i] = qo_gguf_value(b, enc, i);
      return 0;
    case QO_ENC_IQ3_S: {  // :350-361: signed grid bytes (SignedIQ3Grid, :594-605), then q * (d * scale) per 32
      int8_t quants[256];
      for (int i = 0; i < 64; ++i) {
        const int grid = b[2 + i] | (((b[66 + i / 8] >> (i % 8)) & 1) << 8);
        const int signs = (b[74 + i / 2] >> ((i & 1) * 4)) & 15;
        for (int t = 0; t < 4; ++t) {
          const int q = int((kG3S.v[grid] >> (t * 8)) & 255);
          quants[i * 4 + t] = int8_t((signs >> t) & 1 ? -q : q);
        }
      }
      const float d = half_at(b);
      for (int g = 0; g < 8; ++g) {
        const float sc = d * float(1 + 2 * ((b[106 + g / 2] >> ((g & 1) * 4)) & 15));
        for (int i = 0; i < 32; ++i) out[g * 32 + i] = float(quants[g * 32 + i]) * sc;
      }
      return 0;
    }
    case QO_ENC_Q5_K: {  // :296-312 with DecodeBits (:30-66): q = low4 | high1 << 4, cvt(q) * Scale + Bias
      float d = half_at(b), dm = half_at(b + 2);
      for (int g = 0; g < 8; ++g) {
        int scale, minimum;
        if (g < 4) { scale = b[4 + g] & 63; minimum = b[8 + g] & 63; }
        else { scale = (b[8 + g] & 15) | ((b[g] >> 6) << 4); minimum = (b[8 + g] >> 4) | ((b[4 + g] >> 6) << 4); }
        const float s = d * float(scale), bias = -(dm * float(minimum));
        const uint8_t *low = b + 48 + (g / 2) * 32, *high = b + 16;
        for (int i = 0; i < 32; ++i) {
          const int q = ((low[i] >> ((g & 1) * 4)) & 15) | (((high[i] >> g) & 1) << 4);
          out[g * 32 + i] = float(q) * s + bias;
        }
      }
      return 0;
    }
    case QO_ENC_IQ4_NL:  // :338
      decode_iq4(b + 2, out, half_at(b));
      return 0;
    case QO_ENC_IQ4_XS: {  // :339-348
      const float d = half_at(b);
      for (int g = 0; g < 8; ++g) {
        const int scale = (((b[4 + g / 2] >> ((g & 1) * 4)) & 15) | ((((int(b[2]) | (int(b[3]) << 8)) >> (g * 2)) & 3) << 4)) - 32;
        decode_iq4(b + 8 + g * 16, out + g * 32, d * float(scale));
      }
      return 0;
    }
    case QO_ENC_Q8_0: {  // DecodeSigned32 (:68-83)
      __m256 d = _mm256_set1_ps(half_at(b));
      for (int c = 0; c < 4; ++c) {
        __m128i v = _mm_loadl_epi64(reinterpret_cast<const __m128i *>(b + 2 + c * 8));
        __m256 q = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(v));
        _mm256_storeu_ps(out + c * 8, _mm256_mul_ps(q, d));
      }
      return 0;
    }
    case QO_ENC_Q2_K:  // per element GGUFValue (:294-295)
      for (int i = 0; i < 256; ++i) out[i] = qo_gguf_value(b, enc, i);
      return 0;
    case QO_ENC_Q4_K: {  // :296-312 + DecodeLow4 (:7-28)
      float d = half_at(b), dm = half_at(b + 2);
      for (int g = 0; g < 8; ++g) {
        int scale, minimum;
        if (g < 4) { scale = b[4 + g] & 63; minimum = b[8 + g] & 63; }
        else { scale = (b[8 + g] & 15) | ((b[g] >> 6) << 4); minimum = (b[8 + g] >> 4) | ((b[4 + g] >> 6) << 4); }
        __m256 s = _mm256_set1_ps(d * float(scale));
        __m256 bias = _mm256_set1_ps(-(dm * float(minimum)));
        const uint8_t *low = b + 16 + (g / 2) * 32;
        __m128i shift = _mm_cvtsi32_si128((g & 1) * 4);
        for (int c = 0; c < 4; ++c) {
          __m256i q = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(low + c * 8), shift), _mm256_set1_epi32(15));
          __m256 v = _mm256_add_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(q), s), bias);
          _mm256_storeu_ps(out + g * 32 + c * 8, v);
        }
      }
      return 0;
    }
    case QO_ENC_Q6_K:
    case QO_ENC_Q3_K: {  // :313-337 + DecodeBits (:30-66)
      bool q6 = enc == QO_ENC_Q6_K;
      float d = q6 ? half_at(b + 208) : half_at(b + 108);
      int low_mask = q6 ? 15 : 3, high_mask = q6 ? 3 : 1, high_left = q6 ? 4 : 2, center = q6 ? 32 : 4;
      for (int g = 0; g < 16; ++g) {
        int part = g / 8, quarter = (g % 8) / 2, lane = (g & 1) * 16;
        int scale, low_shift, high_shift;
        const uint8_t *low, *high;
        if (q6) {
          scale = signed_byte(b[192 + g]);
          low = b + part * 64 + (quarter & 1) * 32 + lane;
          high = b + 128 + part * 32 + lane;
          low_shift = (quarter / 2) * 4;
          high_shift = quarter * 2;
        } else {
          scale = (((b[96 + g % 8] >> ((g / 8) * 4)) & 15) | (((b[104 + g % 4] >> ((g / 4) * 2)) & 3) << 4)) - 32;
          low = b + 32 + part * 32 + lane;
          high = b + lane;
          low_shift = quarter * 2;
          high_shift = g / 2;
        }
        __m256 s = _mm256_set1_ps(d * float(scale));
        __m256 bias = _mm256_set1_ps(0.0f);
        for (int c = 0; c < 2; ++c) {
          __m256i lo = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(low + c * 8), _mm_cvtsi32_si128(low_shift)), _mm256_set1_epi32(low_mask));
          __m256i hi = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(high + c * 8), _mm_cvtsi32_si128(high_shift)), _mm256_set1_epi32(high_mask));
          hi = _mm256_sll_epi32(hi, _mm_cvtsi32_si128(high_left));
          __m256i q = _mm256_sub_epi32(_mm256_or_si256(lo, hi), _mm256_set1_epi32(center));
          __m256 v = _mm256_add_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(q), s), bias);
          _mm256_storeu_ps(out + g * 16 + c * 8, v);
        }
      }
      return 0;
    }
  }
  return -1;
}

int qo_gguf_dequantize(const uint8_t *data, int enc, int64_t count, float *out) {  // :370-383
  int elements = qo_gguf_block_elements(enc), bytes = qo_gguf_block_bytes(enc);
  if (elements < 0 || count < 0) return -1;
  int64_t offset = 0;
  while (count - offset >= elements) {
    qo_gguf_decode_block(data + (offset / elements) * bytes, enc, out + offset);
    offset += elements;
  }
  for (int64_t i = offset; i < count; ++i) out[i] = qo_gguf_value(data, enc, i);
  return 0;
}

// readGGUF4 (src/backends/vulkan/shaders/gguf.glsl:591-655) reads the packed
// buffer as 32-bit words; packedWord (:582-586) assembles 4 bytes at any
// offset.  Four adjacent values share block metadata; index % 4 == 0.
static uint32_t packed_byte(const uint8_t *data, uint64_t off) { return data[off]; }
static uint32_t packed_word(const uint8_t *data, uint64_t off) {
  return data[off] | (uint32_t(data[off + 1]) << 8) | (uint32_t(data[off + 2]) << 16) | (uint32_t(data[off + 3]) << 24);
}
static float packed_half(const uint8_t *data, uint64_t off) { return half_at(data + off); }

// readGGUF (gguf.glsl:477-512) for encodings 10-13: one value.
static float shader_read(const uint8_t *data, int enc, uint64_t index) {
  if (enc == QO_ENC_IQ3_XXS) {  // :478-485
    const uint64_t base = (index / 256u) * 98u;
    const uint32_t i = uint32_t(index & 255u), group = i / 32u;
    const uint32_t bits = packed_word(data, base + 66u + group * 4u);
    const uint32_t signs = kSigns.v[(bits >> (7u * ((i % 32u) / 8u))) & 127u];
    int q = int((kG3XXS.v[packed_byte(data, base + 2u + i / 4u)] >> ((i % 4u) * 8u)) & 255u);
    if (signs & (1u << (i % 8u))) q = -q;
    return (packed_half(data, base) * (0.5f + float(bits >> 28u)) * 0.5f) * float(q);
  }
  if (enc == QO_ENC_Q2_0) {  // :486-490
    const uint64_t base = (index / 64u) * 18u, i = index % 64u;
    return packed_half(data, base) * float(int((packed_byte(data, base + 2u + i / 4u) >> ((i % 4u) * 2u)) & 3u) - 1);
  }
  // IQ2_XXS / IQ2_S (:491-512)
  const uint32_t i = uint32_t(index & 255u), group = i / 32u, lane = (i % 32u) / 8u;
  const uint64_t base = (index / 256u) * (enc == QO_ENC_IQ2_XXS ? 66u : 82u);
  uint64_t grid;
  uint32_t signs;
  float delta;
  if (enc == QO_ENC_IQ2_XXS) {
    const uint32_t word = packed_word(data, base + 6u + group * 8u);
    grid = kG2XXS.v[packed_byte(data, base + 2u + group * 8u + lane)];
    signs = kSigns.v[(word >> (7u * lane)) & 127u];
    delta = packed_half(data, base) * (0.5f + float(word >> 28u)) * 0.25f;
  } else {
    grid = kG2S.v[packed_byte(data, base + 2u + group * 4u + lane) |
                  (((packed_byte(data, base + 66u + group) >> (lane * 2u)) & 3u) << 8u)];
    signs = packed_byte(data, base + 34u + i / 8u);
    const uint32_t scale = (packed_byte(data, base + 74u + group) >> (((i % 32u) / 16u) * 4u)) & 15u;
    delta = packed_half(data, base) * (0.5f + float(scale)) * 0.25f;
  }
  int q = int((grid >> ((i % 8u) * 8u)) & 255u);
  if (signs & (1u << (i % 8u))) q = -q;
  return delta * float(q);
}

int qo_gguf_read4(const uint8_t *data, int enc, int64_t index, float *o) {
  if (index % 4) return -1;
  if (enc == QO_ENC_Q2_0 || enc == QO_ENC_IQ2_XXS || enc == QO_ENC_IQ2_S || enc == QO_ENC_IQ3_XXS) {
    for (int t = 0; t < 4; ++t) o[t] = shader_read(data, enc, uint64_t(index) + t);  // :592 (encodings >= 10)
    return 0;
  }
  if (enc == QO_ENC_IQ3_S) {  // :648-655 (readGGUF4's last case)
    const uint64_t base = (uint64_t(index) >> 8) * 110u;
    const uint32_t item = uint32_t(index) & 255u, group = item / 32u;
    const uint32_t grid = packed_byte(data, base + 2u + item / 4u) |
                          (((packed_byte(data, base + 66u + group) >> ((item % 32u) / 4u)) & 1u) << 8);
    const uint32_t sb = packed_byte(data, base + 74u + item / 8u);
    const uint32_t scale = 1u + 2u * ((packed_byte(data, base + 106u + group / 2u) >> ((group % 2u) * 4u)) & 15u);
    const float a = packed_half(data, base) * float(scale);
    for (int t = 0; t < 4; ++t) {
      int q = int((kG3S.v[grid] >> (8 * t)) & 255u);
      if ((sb >> (uint32_t(t) + (item & 4u))) & 1u) q = -q;
      o[t] = a * float(q);
    }
    return 0;
  }
  uint64_t idx = uint64_t(index);
  uint32_t item = idx & 255u, lane = item & 31u, group = item >> 5u;
  if (enc == QO_ENC_Q2_K) {
    uint64_t base = (idx >> 8) * 84u;
    uint32_t sc = packed_byte(data, base + (item >> 4));
    uint32_t w = packed_word(data, base + 16u + (item >> 7) * 32u + (item & 31u));
    float a = packed_half(data, base + 80u) * float(sc & 15u);
    float m = packed_half(data, base + 82u) * float(sc >> 4);
    for (int t = 0; t < 4; ++t) o[t] = a * float(((w >> (8 * t)) >> (((item & 127u) >> 5) * 2u)) & 3u) - m;
    return 0;
  }
  if (enc == QO_ENC_Q8_0) {
    uint64_t base = (idx >> 5) * 34u;
    uint32_t w = packed_word(data, base + 2u + (idx & 31u));
    float d = packed_half(data, base);
    for (int t = 0; t < 4; ++t) o[t] = d * float(signed_byte(uint8_t(w >> (8 * t))));
    return 0;
  }
  if (enc == QO_ENC_Q4_K || enc == QO_ENC_Q5_K) {  // :605-617
    const bool q5 = enc == QO_ENC_Q5_K;
    uint64_t base = (idx >> 8) * (q5 ? 176u : 144u);
    uint32_t scale, minimum;
    if (group < 4) {
      scale = packed_byte(data, base + 4u + group) & 63u;
      minimum = packed_byte(data, base + 8u + group) & 63u;
    } else {
      scale = (packed_byte(data, base + 8u + group) & 15u) | ((packed_byte(data, base + group) >> 6) << 4);
      minimum = (packed_byte(data, base + 8u + group) >> 4) | ((packed_byte(data, base + 4u + group) >> 6) << 4);
    }
    uint32_t w = packed_word(data, base + (q5 ? 48u : 16u) + (item >> 6) * 32u + lane);
    uint32_t hw = q5 ? packed_word(data, base + 16u + lane) : 0u;
    float a = packed_half(data, base) * float(scale);
    float m = packed_half(data, base + 2u) * float(minimum);
    for (int t = 0; t < 4; ++t) {
      uint32_t q = ((w >> (8 * t)) >> ((group & 1u) * 4u)) & 15u;
      if (q5) q |= ((((hw >> (8 * t)) & 255u) >> group) & 1u) << 4;
      o[t] = a * float(q) - m;
    }
    return 0;
  }
  if (enc == QO_ENC_IQ4_NL) {  // :636-640
    uint64_t base = (idx >> 5) * 18u;
    uint32_t i = uint32_t(idx & 31u);
    uint32_t w = packed_word(data, base + 2u + i % 16u);
    float d = packed_half(data, base);
    for (int t = 0; t < 4; ++t) o[t] = d * float(kIQ4[(((w >> (8 * t)) & 255u) >> ((i / 16u) * 4u)) & 15u]);
    return 0;
  }
  if (enc == QO_ENC_IQ4_XS) {  // :641-647
    uint64_t base = (idx >> 8) * 136u;
    uint32_t scale = ((packed_byte(data, base + 4u + group / 2u) >> ((group % 2u) * 4u)) & 15u) |
                     ((((packed_byte(data, base + 2u) | (packed_byte(data, base + 3u) << 8)) >> (group * 2u)) & 3u) << 4);
    uint32_t w = packed_word(data, base + 8u + group * 16u + item % 16u);
    float a = packed_half(data, base) * float(int(scale) - 32);
    for (int t = 0; t < 4; ++t) o[t] = a * float(kIQ4[(((w >> (8 * t)) & 255u) >> (((item % 32u) / 16u) * 4u)) & 15u]);
    return 0;
  }
  if (enc == QO_ENC_Q6_K) {
    uint64_t base = (idx >> 8) * 210u;
    uint32_t part = item >> 7, quarter = (item & 127u) >> 5;
    uint32_t lo = packed_word(data, base + part * 64u + (quarter & 1u) * 32u + lane);
    uint32_t hi = packed_word(data, base + 128u + part * 32u + lane);
    int scale = signed_byte(uint8_t(packed_byte(data, base + 192u + (item >> 4))));
    float a = packed_half(data, base + 208u) * float(scale);
    for (int t = 0; t < 4; ++t) {
      uint32_t l = (lo >> (8 * t)) & 255u, h = (hi >> (8 * t)) & 255u;
      int q = int(((l >> ((quarter >> 1) * 4u)) & 15u) | (((h >> (quarter * 2u)) & 3u) << 4)) - 32;
      o[t] = a * float(q);
    }
    return 0;
  }
  if (enc == QO_ENC_Q3_K) {
    uint64_t base = (idx >> 8) * 110u;
    uint32_t g = item >> 4;
    uint32_t scale = ((packed_byte(data, base + 96u + g % 8u) >> ((g / 8u) * 4u)) & 15u) |
                     (((packed_byte(data, base + 104u + g % 4u) >> ((g / 4u) * 2u)) & 3u) << 4);
    uint32_t qs = packed_word(data, base + 32u + (item / 128u) * 32u + lane);
    uint32_t hm = packed_word(data, base + lane);
    float a = packed_half(data, base + 108u) * float(int(scale) - 32);
    for (int t = 0; t < 4; ++t) {
      int q = int((((qs >> (8 * t)) & 255u) >> (((item % 128u) / 32u) * 2u)) & 3u);
      bool high = ((((hm >> (8 * t)) & 255u) >> (item / 32u)) & 1u) != 0;
      q -= high ? 0 : 4;
      o[t] = a * float(q);
    }
    return 0;
  }
  return -1;
}

// ===========================================================================
// AVX2 dots
// ===========================================================================

// VectorDot (src/backends/cpu/QuickNN.CPU.Inference.AVX2.inc:7-67).
float qo_vector_dot(int count, const float *a, const float *b) {
  __m256 y0 = _mm256_setzero_ps(), y1 = y0, y2 = y0, y3 = y0;
  int n32 = count >> 5;
  for (int i = 0; i < n32; ++i, a += 32, b += 32) {
    y0 = _mm256_add_ps(y0, _mm256_mul_ps(_mm256_loadu_ps(a), _mm256_loadu_ps(b)));
    y1 = _mm256_add_ps(y1, _mm256_mul_ps(_mm256_loadu_ps(a + 8), _mm256_loadu_ps(b + 8)));
    y2 = _mm256_add_ps(y2, _mm256_mul_ps(_mm256_loadu_ps(a + 16), _mm256_loadu_ps(b + 16)));
    y3 = _mm256_add_ps(y3, _mm256_mul_ps(_mm256_loadu_ps(a + 24), _mm256_loadu_ps(b + 24)));
  }
  y0 = _mm256_add_ps(y0, y1);
  y2 = _mm256_add_ps(y2, y3);
  y0 = _mm256_add_ps(y0, y2);
  int n8 = (count & 31) >> 3;
  for (int i = 0; i < n8; ++i, a += 8, b += 8)
    y0 = _mm256_add_ps(y0, _mm256_mul_ps(_mm256_loadu_ps(a), _mm256_loadu_ps(b)));
  float r = hreduce(y0);
  for (int i = 0; i < (count & 7); ++i) r = r + a[i] * b[i];
  return r;
}

// Int4VectorDot (src/backends/cpu/QuickNN.CPU.Inference.AVX2.inc:210-285):
// per element t = cvt(n-8)*s, t = t*x, acc += t; 8 lanes; scalar tail.
float qo_int4_vector_dot(int count, const float *x, const uint8_t *w) {
  const __m256i shifts = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
  const __m256i mask = _mm256_set1_epi32(15), center = _mm256_set1_epi32(8);
  __m256 acc = _mm256_setzero_ps();
  int groups = count >> 5;
  for (int g = 0; g < groups; ++g, w += 20, x += 32) {
    float sf;
    std::memcpy(&sf, w, 4);
    __m256 s = _mm256_set1_ps(sf);
    for (int c = 0; c < 4; ++c) {
      uint32_t word;
      std::memcpy(&word, w + 4 + c * 4, 4);
      __m256i q = _mm256_sub_epi32(_mm256_and_si256(_mm256_srlv_epi32(_mm256_set1_epi32(int(word)), shifts), mask), center);
      __m256 t = _mm256_mul_ps(_mm256_cvtepi32_ps(q), s);
      t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
      acc = _mm256_add_ps(acc, t);
    }
  }
  float r = hreduce(acc);
  int tail = count & 31;
  if (tail) {
    float sf;
    std::memcpy(&sf, w, 4);
    for (int i = 0; i < tail; ++i) {
      int n = (w[4 + i / 2] >> ((i & 1) * 4)) & 15;
      float t = float(n - 8) * sf;
      t = t * x[i];
      r = r + t;
    }
  }
  return r;
}

// PackedDotQ8 (src/io/QuickNN.GGUF.Dot.AVX2.inc:330-368).
static float packed_dot_q8(const uint8_t *b, const float *x, int blocks) {
  __m256 acc = _mm256_setzero_ps();
  for (int blk = 0; blk < blocks; ++blk, b += 34, x += 32) {
    __m256 d = _mm256_set1_ps(half_at(b));
    for (int c = 0; c < 4; ++c) {
      __m128i v = _mm_loadl_epi64(reinterpret_cast<const __m128i *>(b + 2 + c * 8));
      __m256 t = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(v)), d);
      t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
      acc = _mm256_add_ps(acc, t);
    }
  }
  return hreduce(acc);
}

// PackedDotQ4K (src/io/QuickNN.GGUF.Dot.AVX2.inc:9-111): two accumulators,
// chunks 0,2 -> ymm0 and 1,3 -> ymm12; w = cvt(q)*(sc*d) - (m*dmin).
static float packed_dot_q4k(const uint8_t *b, const float *x, int blocks) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  const __m256i mask = _mm256_set1_epi32(15);
  for (int blk = 0; blk < blocks; ++blk, b += 144) {
    float d = half_at(b), dm = half_at(b + 2);
    for (int g = 0; g < 8; ++g, x += 32) {
      int sc, m;
      if (g < 4) { sc = b[4 + g] & 63; m = b[8 + g] & 63; }
      else { sc = ((b[g] >> 6) << 4) | (b[8 + g] & 15); m = ((b[4 + g] >> 6) << 4) | (b[8 + g] >> 4); }
      __m256 s = _mm256_mul_ps(_mm256_set1_ps(float(sc)), _mm256_set1_ps(d));
      __m256 mm = _mm256_mul_ps(_mm256_set1_ps(float(m)), _mm256_set1_ps(dm));
      const uint8_t *q = b + 16 + (g >> 1) * 32;
      __m128i shift = _mm_cvtsi32_si128((g & 1) * 4);
      for (int c = 0; c < 4; ++c) {
        __m256i v = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(q + c * 8), shift), mask);
        __m256 t = _mm256_sub_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(v), s), mm);
        t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
        if (c & 1) acc1 = _mm256_add_ps(acc1, t);
        else acc0 = _mm256_add_ps(acc0, t);
      }
    }
  }
  return hreduce(_mm256_add_ps(acc0, acc1));
}

// PackedDotQ6K (src/io/QuickNN.GGUF.Dot.AVX2.inc:423-513).
static float packed_dot_q6k(const uint8_t *b, const float *x, int blocks) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  const __m256i m15 = _mm256_set1_epi32(15), m3 = _mm256_set1_epi32(3), c32 = _mm256_set1_epi32(32);
  for (int blk = 0; blk < blocks; ++blk, b += 210) {
    __m256 d = _mm256_set1_ps(half_at(b + 208));
    for (int g = 0; g < 16; ++g, x += 16) {
      __m256 s = _mm256_mul_ps(_mm256_set1_ps(float(signed_byte(b[192 + g]))), d);
      int quarter = (g >> 1) & 3;
      __m128i lshift = _mm_cvtsi32_si128((quarter >> 1) << 2), hshift = _mm_cvtsi32_si128(quarter << 1);
      const uint8_t *lo = b + ((g >> 3) << 6) + (((g >> 1) & 1) << 5) + ((g & 1) << 4);
      const uint8_t *hi = b + 128 + ((g >> 3) << 5) + ((g & 1) << 4);
      for (int c = 0; c < 2; ++c) {
        __m256i l = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(lo + c * 8), lshift), m15);
        __m256i h = _mm256_slli_epi32(_mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(hi + c * 8), hshift), m3), 4);
        __m256i q = _mm256_sub_epi32(_mm256_or_si256(l, h), c32);
        __m256 t = _mm256_mul_ps(_mm256_cvtepi32_ps(q), s);
        t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
        if (c) acc1 = _mm256_add_ps(acc1, t);
        else acc0 = _mm256_add_ps(acc0, t);
      }
    }
  }
  return hreduce(_mm256_add_ps(acc0, acc1));
}

// PackedDotQ3K (src/io/QuickNN.GGUF.Dot.AVX2.inc:515-613).
static float packed_dot_q3k(const uint8_t *b, const float *x, int blocks) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  const __m256i m3 = _mm256_set1_epi32(3), m1 = _mm256_set1_epi32(1), c4 = _mm256_set1_epi32(4);
  for (int blk = 0; blk < blocks; ++blk, b += 110) {
    __m256 d = _mm256_set1_ps(half_at(b + 108));
    for (int g = 0; g < 16; ++g, x += 16) {
      int sc = ((b[96 + (g & 7)] >> ((g >> 3) << 2)) & 15) | (((b[104 + (g & 3)] >> ((g >> 2) << 1)) & 3) << 4);
      __m256 s = _mm256_mul_ps(_mm256_set1_ps(float(sc - 32)), d);
      __m128i hshift = _mm_cvtsi32_si128(g >> 1), lshift = _mm_cvtsi32_si128(((g >> 1) & 3) << 1);
      const uint8_t *lo = b + 32 + ((g >> 3) << 5) + ((g & 1) << 4);
      const uint8_t *hm = b + ((g & 1) << 4);
      for (int c = 0; c < 2; ++c) {
        __m256i l = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(lo + c * 8), lshift), m3);
        __m256i h = _mm256_slli_epi32(_mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(hm + c * 8), hshift), m1), 2);
        __m256i q = _mm256_sub_epi32(_mm256_or_si256(l, h), c4);
        __m256 t = _mm256_mul_ps(_mm256_cvtepi32_ps(q), s);
        t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
        if (c) acc1 = _mm256_add_ps(acc1, t);
        else acc0 = _mm256_add_ps(acc0, t);
      }
    }
  }
  return hreduce(_mm256_add_ps(acc0, acc1));
}

// PackedDotQ5K (src/io/QuickNN.GGUF.Dot.AVX2.inc:113-236): PackedDotQ4K with
// the quants at 48 and the fifth bit of element i from byte 16 + i % 32,
// shifted by the sub-block index.
static float packed_dot_q5k(const uint8_t *b, const float *x, int blocks) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  const __m256i mask = _mm256_set1_epi32(15), one = _mm256_set1_epi32(1);
  for (int blk = 0; blk < blocks; ++blk, b += 176) {
    float d = half_at(b), dm = half_at(b + 2);
    for (int g = 0; g < 8; ++g, x += 32) {
      int sc, m;
      if (g < 4) { sc = b[4 + g] & 63; m = b[8 + g] & 63; }
      else { sc = ((b[g] >> 6) << 4) | (b[8 + g] & 15); m = ((b[4 + g] >> 6) << 4) | (b[8 + g] >> 4); }
      __m256 s = _mm256_mul_ps(_mm256_set1_ps(float(sc)), _mm256_set1_ps(d));
      __m256 mm = _mm256_mul_ps(_mm256_set1_ps(float(m)), _mm256_set1_ps(dm));
      const uint8_t *q = b + 48 + (g >> 1) * 32;
      __m128i shift = _mm_cvtsi32_si128((g & 1) * 4), hshift = _mm_cvtsi32_si128(g);
      for (int c = 0; c < 4; ++c) {
        __m256i v = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(q + c * 8), shift), mask);
        __m256i h = _mm256_and_si256(_mm256_srl_epi32(load_u8x8_epi32(b + 16 + c * 8), hshift), one);
        v = _mm256_or_si256(v, _mm256_slli_epi32(h, 4));
        __m256 t = _mm256_sub_ps(_mm256_mul_ps(_mm256_cvtepi32_ps(v), s), mm);
        t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
        if (c & 1) acc1 = _mm256_add_ps(acc1, t);
        else acc0 = _mm256_add_ps(acc0, t);
      }
    }
  }
  return hreduce(_mm256_add_ps(acc0, acc1));
}

// The codebook values of 8 nibbles as floats (vpshufb of the 16-byte table,
// vpmovsxbd, vcvtdq2ps).
static __m256 iq4_8(const uint8_t *src, int hi) {
  int v[8];
  for (int j = 0; j < 8; ++j) v[j] = kIQ4[(src[j] >> (hi * 4)) & 15];
  return _mm256_cvtepi32_ps(_mm256_setr_epi32(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]));
}

// PackedDotIQ4XS (Dot.AVX2.inc:238-328): per sub-block s = d * (sc - 32); per
// 8 elements t = cvt(code) * s, t = t * x; pieces alternate between two
// accumulators (elements 0-7, 16-23 in the first; 8-15, 24-31 in the second).
static float packed_dot_iq4xs(const uint8_t *b, const float *x, int blocks) {
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  for (int blk = 0; blk < blocks; ++blk, b += 136) {
    const float d = half_at(b);
    for (int g = 0; g < 8; ++g, x += 32) {
      const int sc = (((b[4 + g / 2] >> ((g & 1) * 4)) & 15) | ((((int(b[2]) | (int(b[3]) << 8)) >> (g * 2)) & 3) << 4)) - 32;
      const __m256 s = _mm256_mul_ps(_mm256_set1_ps(float(sc)), _mm256_set1_ps(d));
      const uint8_t *q = b + 8 + g * 16;
      for (int c = 0; c < 4; ++c) {  // low nibbles 0-7, 8-15, then high nibbles 16-23, 24-31
        __m256 t = _mm256_mul_ps(iq4_8(q + (c & 1) * 8, c >> 1), s);
        t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
        if (c & 1) acc1 = _mm256_add_ps(acc1, t);
        else acc0 = _mm256_add_ps(acc0, t);
      }
    }
  }
  return hreduce(_mm256_add_ps(acc0, acc1));
}

// PackedDotIQ4NL (Dot.AVX2.inc:370-421): one accumulator; per 8 elements
// t = cvt(code) * d, t = t * x, acc += t.
static float packed_dot_iq4nl(const uint8_t *b, const float *x, int blocks) {
  __m256 acc = _mm256_setzero_ps();
  for (int blk = 0; blk < blocks; ++blk, b += 18, x += 32) {
    const __m256 d = _mm256_set1_ps(half_at(b));
    for (int c = 0; c < 4; ++c) {
      __m256 t = _mm256_mul_ps(iq4_8(b + 2 + (c & 1) * 8, c >> 1), d);
      t = _mm256_mul_ps(t, _mm256_loadu_ps(x + c * 8));
      acc = _mm256_add_ps(acc, t);
    }
  }
  return hreduce(acc);
}

// GGUFTryDot (src/io/QuickNN.GGUF.Quantization.pas:255-272) for the formats
// in scope; returns NaN where the reference returns False (Q2_K, partial
// super-blocks), leaving the caller to decode + VectorDot.
static bool try_dot(const uint8_t *data, int enc, const float *x, int count, float &value) {
  if (count < 32 || count % 32 != 0) return false;
  if (enc != QO_ENC_Q8_0 && enc != QO_ENC_IQ4_NL && count % 256 != 0) return false;
  switch (enc) {
    case QO_ENC_Q8_0: value = packed_dot_q8(data, x, count / 32); return true;
    case QO_ENC_Q6_K: value = packed_dot_q6k(data, x, count / 256); return true;
    case QO_ENC_Q3_K: value = packed_dot_q3k(data, x, count / 256); return true;
    case QO_ENC_Q4_K: value = packed_dot_q4k(data, x, count / 256); return true;
    case QO_ENC_Q5_K: value = packed_dot_q5k(data, x, count / 256); return true;
    case QO_ENC_IQ4_NL: value = packed_dot_iq4nl(data, x, count / 32); return true;
    case QO_ENC_IQ4_XS: value = packed_dot_iq4xs(data, x, count / 256); return true;
  }
  return false;
}

float qo_packed_dot(const uint8_t *data, int enc, const float *x, int count) {
  float v;
  if (try_dot(data, enc, x, count, v)) return v;
  return std::nanf("");
}

// ===========================================================================
// TCPUProjection.Linear (src/backends/cpu/QuickNN.CPU.Inference.pas:316-428)
// ===========================================================================
void *qo_pool_create(int threads) {
  if (threads < 0 || threads > 64) return nullptr;  // :112
  if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("f16c")) return nullptr;
  if (threads == 0) threads = int(std::min(8u, std::max(1u, std::thread::hardware_concurrency())));  // :114
  return new Pool(std::max(1, threads));
}
void qo_pool_destroy(void *pool) { delete static_cast<Pool *>(pool); }
int qo_pool_threads(void *pool) { return static_cast<Pool *>(pool)->threads; }

static int64_t row_bytes_for(int enc, int in_dim) {
  if (enc == QO_ENC_INT4) return qo_int4_row_bytes(in_dim);
  int e = qo_gguf_block_elements(enc);
  if (e < 0 || in_dim % e) return -1;
  return int64_t(in_dim / e) * qo_gguf_block_bytes(enc);
}

int qo_cpu_linear(void *pool_, const uint8_t *w, int enc, const float *x, float *y, int in_dim, int out_dim) {
  Pool *pool = static_cast<Pool *>(pool_);
  if (!pool || !w || !x || !y || in_dim < 1 || out_dim < 1) return -1;
  int64_t row_bytes = row_bytes_for(enc, in_dim);
  if (row_bytes < 0) return -1;
  int threads = ((int64_t)in_dim * out_dim >= 1048576) ? pool->threads : 1;  // :378-379
  auto job = [&](int index) {
    std::vector<float> scratch;
    for (int64_t r = (int64_t)out_dim * index / threads; r < (int64_t)out_dim * (index + 1) / threads; ++r) {
      const uint8_t *row = w + r * row_bytes;
      if (enc == QO_ENC_INT4) { y[r] = qo_int4_vector_dot(in_dim, x, row); continue; }  // :402-403
      float v;
      if (try_dot(row, enc, x, in_dim, v)) { y[r] = v; continue; }  // :396
      if (scratch.empty()) scratch.resize(size_t((in_dim + 31) / 32) * 32);
      qo_gguf_dequantize(row, enc, in_dim, scratch.data());  // :407-408
      y[r] = qo_vector_dot(in_dim, x, scratch.data());       // :424
    }
  };
  if (threads == 1) job(0);
  else pool->run(job);
  return 0;
}

// ===========================================================================
// Decode-layer composites: src/models/QuickNN.Models.QwenHybrid.CPU.pas
// ===========================================================================

// Normalize (:110-120): double sum of squares, Single inverse, x*inv*(g+add_one).
int qo_rmsnorm(const float *x, const float *gamma, int rows, int dim, float eps, int add_one, float *out) {
  if (!x || !out || rows < 1 || dim < 1) return -1;
  for (int h = 0; h < rows; ++h) {
    double sum = 0;
    for (int j = 0; j < dim; ++j) sum = sum + double(x[h * dim + j]) * double(x[h * dim + j]);
    float inv = float(1.0 / std::sqrt(sum / dim + double(eps)));
    for (int j = 0; j < dim; ++j) {
      float g = (gamma ? gamma[j] : 0.0f) + float(add_one ? 1 : 0);
      out[h * dim + j] = x[h * dim + j] * inv * g;
    }
  }
  return 0;
}

// Sigmoid (:78-82) and the clamped SiLU of Step (:242-246).
static float sigmoid(float x) {
  if (x >= 0) return float(1.0 / (1.0 + std::exp(-double(x))));
  double e = std::exp(double(x));
  return float(e / (1.0 + e));
}
float qo_silu(float g) {
  if (g <= -20) return 0.0f;
  if (g < 20) return g * sigmoid(g);
  return g;
}

// Step's MLP (:238-248): gate, up, silu(gate)*up, down -- one token at a time.
int qo_cpu_mlp(void *pool, const uint8_t *gate, const uint8_t *up, const uint8_t *down, int enc, const float *x,
               int rows, int hidden, int inter, float *out) {
  std::vector<float> g(inter), u(inter);
  for (int r = 0; r < rows; ++r) {
    int rc = qo_cpu_linear(pool, gate, enc, x + (size_t)r * hidden, g.data(), hidden, inter);
    rc |= qo_cpu_linear(pool, up, enc, x + (size_t)r * hidden, u.data(), hidden, inter);
    if (rc) return -1;
    for (int j = 0; j < inter; ++j) g[j] = qo_silu(g[j]) * u[j];
    if (qo_cpu_linear(pool, down, enc, g.data(), out + (size_t)r * hidden, inter, hidden)) return -1;
  }
  return 0;
}

// ===========================================================================
// MoE
// ===========================================================================

// GO_MOE_ROUTE (src/backends/vulkan/shaders/moe.comp:25-50): softmax over the
// experts, k rounds of argmax over the probabilities with ties to the lower id
// (:36-46), the selected entry set to -1, optional renormalisation by the
// rank-ordered sum of the top-k (:47-48).
//  - v_e = exp(l_e - max) (:31): the shader's exp has implementation-defined
//    precision; here it is the correctly rounded fp32 exponential (double exp,
//    rounded once).
//  - The denominator follows sumGroup (:20, :32): 256 partial sums, partial L
//    over experts L, L+256, ... in ascending id (:31), then the LDS tree
//    partial[L] += partial[L+s] for s = 128 .. 1.
//  - p_e = v_e / denominator (:33), so distinct logits whose probabilities
//    round equal tie, and the lower id wins.
// select_on_logits=1 ranks by logit instead (the same order wherever no two
// distinct probabilities round equal).
int qo_moe_route(const float *logits, int rows, int experts, int k, int normalize, int select_on_logits,
                 uint32_t *ids, float *probs) {
  if (!logits || !ids || !probs || rows < 1 || experts < 1 || k < 1 || k > experts || k > 64) return -1;
  std::vector<float> p(experts), key(experts);
  for (int row = 0; row < rows; ++row) {
    const float *l = logits + (size_t)row * experts;
    float maximum = -3.402823466e38f;
    for (int e = 0; e < experts; ++e) maximum = std::max(maximum, l[e]);
    float partial[256] = {};
    for (int e = 0; e < experts; ++e) {
      p[e] = (float)std::exp((double)(l[e] - maximum));
      partial[e % 256] += p[e];
    }
    for (int s = 128; s > 0; s >>= 1)
      for (int lane = 0; lane < s; ++lane) partial[lane] += partial[lane + s];
    const float denominator = partial[0];
    for (int e = 0; e < experts; ++e) p[e] /= denominator;
    for (int e = 0; e < experts; ++e) key[e] = select_on_logits ? l[e] : p[e];
    std::vector<uint32_t> top_ids(k);
    std::vector<float> top_values(k);
    std::vector<bool> taken(experts, false);
    for (int rank = 0; rank < k; ++rank) {
      float best = 0;
      int best_id = -1;
      for (int e = 0; e < experts; ++e) {
        if (taken[e]) continue;
        if (best_id < 0 || key[e] > best || (key[e] == best && e < best_id)) { best = key[e]; best_id = e; }
      }
      taken[best_id] = true;
      top_ids[rank] = uint32_t(best_id);
      top_values[rank] = p[best_id];
    }
    float total = 0;
    for (int rank = 0; rank < k; ++rank) total += top_values[rank];
    for (int rank = 0; rank < k; ++rank) {
      ids[(size_t)row * k + rank] = top_ids[rank];
      probs[(size_t)row * k + rank] = normalize ? top_values[rank] / total : top_values[rank];
    }
  }
  return 0;
}

// Composed MoE expert layer (TLLMMoE.forward, src/models/QuickNN.Models.LLM.MoE.pas:230-449;
// the reference has no CPU MoE).  Experts run in ascending id order (:412-447);
// each adds p * down(silu(gate x) * (up x)) into the output (moe.comp:70, :125-126).
int qo_cpu_moe(void *pool, const uint8_t *const *gate, const uint8_t *const *up, const uint8_t *const *down,
               const float *x, const uint32_t *ids, const float *probs, int rows, int topk, int hidden, int inter,
               float *out) {
  std::vector<float> g(inter), u(inter), y(hidden);
  for (int r = 0; r < rows; ++r) {
    float *o = out + (size_t)r * hidden;
    for (int j = 0; j < hidden; ++j) o[j] = 0.0f;
    std::vector<std::pair<uint32_t, int>> order;
    for (int t = 0; t < topk; ++t) order.push_back({ids[(size_t)r * topk + t], t});
    std::sort(order.begin(), order.end());
    for (auto &pr : order) {
      uint32_t e = pr.first;
      float p = probs[(size_t)r * topk + pr.second];
      const float *xr = x + (size_t)r * hidden;
      if (qo_cpu_linear(pool, gate[e], QO_ENC_INT4, xr, g.data(), hidden, inter)) return -1;
      if (qo_cpu_linear(pool, up[e], QO_ENC_INT4, xr, u.data(), hidden, inter)) return -1;
      for (int j = 0; j < inter; ++j) g[j] = qo_silu(g[j]) * u[j];
      if (qo_cpu_linear(pool, down[e], QO_ENC_INT4, g.data(), y.data(), inter, hidden)) return -1;
      for (int j = 0; j < hidden; ++j) o[j] = o[j] + y[j] * p;
    }
  }
  return 0;
}

// ===========================================================================
// Multi-row GGUF
// ===========================================================================

// TQNNLinearWeight.Forward GGUF branch (src/core/QuickNN.Quantization.pas:247-258):
// double accumulation over GGUF-decoded weights.  Rows [row_begin,row_end).
int qo_gguf_gemm_scalar(const uint8_t *w, int enc, const float *a, int m, int k, int n, float *c, int row_begin,
                        int row_end) {
  if (row_begin < 0 || row_end > m || k % qo_gguf_block_elements(enc)) return -1;
  std::vector<float> wrow(k);
  int64_t rb = row_bytes_for(enc, k);
  for (int o = 0; o < n; ++o) {
    for (int kk = 0; kk < k; ++kk) wrow[kk] = qo_gguf_value(w + o * rb, enc, kk);
    for (int r = row_begin; r < row_end; ++r) {
      double sum = 0;
      const float *ar = a + (size_t)r * k;
      for (int kk = 0; kk < k; ++kk) sum = sum + double(ar[kk]) * double(wrow[kk]);
      c[(size_t)r * n + o] = float(sum);
    }
  }
  return 0;
}

// ===========================================================================
// The benchmark's int8-activation prefill GEMM (configs[4]: "activations ...
// quantized per 32-element block to int8 for the MFMA path").  The reference
// has no such path (its multi-row GGUF product is the fp32/double one above);
// these restate the rule the HIP kernel applies, so it can be checked bit for
// bit, and the fp32 path above measures what the quantisation costs.
// ===========================================================================

// Per row and 32-element block: the public GGML Q8_0 reference rule
// (quantize_row_q8_0_reference: amax = max|x|, d = amax / 127,
// id = d ? 1/d : 0, q = roundf(x * id)), with d kept in fp32.
// q: [m][k] int8; d: [m][k/32].
int qo_q8_act_quant(const float *a, int m, int k, int8_t *q, float *d) {
  if (!a || !q || !d || m < 1 || k < 32 || k % 32) return -1;
  const int kb = k / 32;
  for (int r = 0; r < m; ++r)
    for (int b = 0; b < kb; ++b) {
      const float *x = a + (size_t)r * k + (size_t)b * 32;
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
      const float dd = amax / 127.0f;
      const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
      for (int i = 0; i < 32; ++i) q[(size_t)r * k + (size_t)b * 32 + i] = int8_t(int(std::roundf(x[i] * id)));
      d[(size_t)r * kb + b] = dd;
    }
  return 0;
}

// C[r][o] = sum over blocks b in ascending order of
//   acc = fma(float(S_b), dx[r][b] * dw[o][b], acc),
// S_b = the exact integer dot of the block's int8 activations and Q8_0 quants,
// dw = the block's fp16 scale (GGUF.Quantization.pas:180-181).  w: Q8_0 rows
// [n][k/32 blocks of 34 B].
int qo_q8_gemm_i8(const uint8_t *w, const int8_t *q, const float *d, int m, int k, int n, float *c) {
  if (!w || !q || !d || !c || m < 1 || n < 1 || k < 32 || k % 32) return -1;
  const int kb = k / 32;
  const size_t rb = (size_t)kb * 34;
  for (int o = 0; o < n; ++o) {
    const uint8_t *wr = w + (size_t)o * rb;
    for (int r = 0; r < m; ++r) {
      float acc = 0.0f;
      for (int b = 0; b < kb; ++b) {
        const uint8_t *blk = wr + (size_t)b * 34;
        const float dw = half_to_float(uint16_t(blk[0] | (blk[1] << 8)));
        const int8_t *xq = q + (size_t)r * k + (size_t)b * 32;
        int32_t s = 0;
        for (int i = 0; i < 32; ++i) s += int32_t(xq[i]) * int32_t(int8_t(blk[2 + i]));
        const float t = d[(size_t)r * kb + b] * dw;
        acc = std::fma(float(s), t, acc);
      }
      c[(size_t)r * n + o] = acc;
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// The rest of a decode layer
// ---------------------------------------------------------------------------

// QwenCPUApplyRoPE (src/models/QuickNN.Models.QwenHybrid.CPU.pas:51-67) with
// RotaryDim = Dim and one position axis: Angle := Pos * Power(Theta, -2*J/Dim)
// in double; X[First] := A*Cos(Angle) - B*Sin(Angle), X[Second] := A*Sin(Angle)
// + B*Cos(Angle) in double, stored as Single.  The rows of a multi-row call sit
// at Position + row (tensor.comp:320).
int qo_rope(float *x, int rows, int heads, int dim, int position, float theta) {
  if (!x || rows < 1 || heads < 1 || dim < 2 || dim % 2 || position < 0 || !(theta > 0.0f)) return -1;
  const int half = dim / 2;
  for (int r = 0; r < rows; ++r)
    for (int h = 0; h < heads; ++h)
      for (int j = 0; j < half; ++j) {
        const double angle = double(position + r) * std::pow(double(theta), -2.0 * double(j) / double(dim));
        float *row = x + ((size_t)r * heads + h) * dim;
        const double a = row[j], b = row[j + half];
        const double c = std::cos(angle), s = std::sin(angle);
        row[j] = float(a * c - b * s);
        row[j + half] = float(a * s + b * c);
      }
  return 0;
}

// The cache layout written by QwenHybrid.CPU.pas:198-204 (and tensor.comp:313-317).
int qo_cache_write(float *cache, const float *k, const float *v, int rows, int kv_heads, int dim, int cap,
                   int position) {
  if (!cache || !k || !v || rows < 1 || kv_heads < 1 || dim < 1 || position < 0 || position + rows > cap) return -1;
  const size_t width = (size_t)kv_heads * dim;
  for (int r = 0; r < rows; ++r)
    for (int h = 0; h < kv_heads; ++h)
      for (int j = 0; j < dim; ++j) {
        const size_t src = (size_t)r * width + (size_t)h * dim + j;
        const size_t t = (size_t)position + r;
        cache[((size_t)h * dim + j) * cap + t] = k[src];
        cache[(size_t)cap * width + ((size_t)h * cap + t) * dim + j] = v[src];
      }
  return 0;
}

// attention.comp:17-44 with mask mode 2 (4 when masked): query row r attends
// to keys [start, position + r] (start = end - window when window > 0 and the
// range is longer), skipping keys whose mask word is zero; scores scaled by
// `scale` or 1/sqrt(dim), optionally capped by softcap * tanh(s / softcap)
// (arguments clamped to +-20); softmax; weighted sum of V.  All in double.
int qo_cached_attention(const float *q, const float *cache, int rows, int cap, int heads, int kv_heads, int dim,
                        int position, int window, float softcap, float scale, int masked, float *out) {
  if (!q || !cache || !out || rows < 1 || cap < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads || dim < 1 ||
      position < 0 || position + rows > cap || window < 0)
    return -1;
  const size_t width = (size_t)kv_heads * dim;
  const float *vbase = cache + (size_t)cap * width;
  const uint32_t *mask = reinterpret_cast<const uint32_t *>(cache + 2 * (size_t)cap * width);
  const int group = heads / kv_heads;
  const double mul = scale > 0.0f ? double(scale) : 1.0 / std::sqrt(double(dim));
  std::vector<double> sc(cap), acc(dim);
  for (int r = 0; r < rows; ++r) {
    const int end = position + r + 1;
    const int start = (window > 0 && end > window) ? end - window : 0;
    for (int h = 0; h < heads; ++h) {
      const int kh = h / group;
      const float *qr = q + ((size_t)r * heads + h) * dim;
      double mx = -INFINITY;
      for (int j = start; j < end; ++j) {
        if (masked && mask[(size_t)r * cap + j] == 0u) {
          sc[j] = -INFINITY;
          continue;
        }
        double s = 0.0;
        for (int d = 0; d < dim; ++d) s += double(qr[d]) * double(cache[((size_t)kh * dim + d) * cap + j]);
        s *= mul;
        if (softcap > 0.0f) s = double(softcap) * std::tanh(std::min(std::max(s / double(softcap), -20.0), 20.0));
        sc[j] = s;
        mx = std::max(mx, s);
      }
      double den = 0.0;
      std::fill(acc.begin(), acc.end(), 0.0);
      for (int j = start; j < end; ++j) {
        if (sc[j] == -INFINITY) continue;
        const double p = std::exp(sc[j] - mx);
        den += p;
        const float *vr = vbase + ((size_t)kh * cap + j) * dim;
        for (int d = 0; d < dim; ++d) acc[d] += p * double(vr[d]);
      }
      float *o = out + ((size_t)r * heads + h) * dim;
      for (int d = 0; d < dim; ++d) o[d] = float(acc[d] / den);
    }
  }
  return 0;
}

namespace {
const float kLowestF = -3.402823466e38f;
bool ranks_before(float s, uint32_t id, float bs, uint32_t bid) { return s > bs || (s == bs && id < bid); }
}  // namespace

// tensor.comp:160-176: k ranks, each the best remaining (score, id) with
// best = -FLT_MAX, id = 0xffffffff to start, penalty applied to seen tokens.
int qo_sample_topk(const float *logits, const uint32_t *seen, int vocab, int k, float penalty, float *scores,
                   uint32_t *ids) {
  if (!logits || !seen || !scores || !ids || vocab < 1 || k < 1 || k > 64) return -1;
  std::vector<uint8_t> used(vocab, 0);
  for (int rank = 0; rank < k; ++rank) {
    float best = kLowestF;
    uint32_t best_id = 0xffffffffu;
    for (int t = 0; t < vocab; ++t) {
      if (seen[t] == 0xffffffffu || used[t]) continue;
      float s = logits[t];
      if (seen[t] != 0u) s = s < 0.0f ? s * penalty : s / penalty;
      if (ranks_before(s, uint32_t(t), best, best_id)) {
        best = s;
        best_id = uint32_t(t);
      }
    }
    if (best_id != 0xffffffffu) used[best_id] = 1;
    scores[rank] = best;
    ids[rank] = best_id;
  }
  return 0;
}

// tensor.comp:177-197: weights exp((v_j - v_0) / T) (fp32, exp correctly
// rounded), the nucleus as the shortest prefix whose running sum reaches
// top_p * total, then the first rank whose running sum exceeds uniform * kept.
uint32_t qo_sample_token(const float *logits, const uint32_t *seen, int vocab, int top_k, float temperature,
                         float top_p, float penalty, float uniform) {
  if (vocab < 1 || top_k < 1 || top_k > 64) return 0xffffffffu;
  const int k = temperature <= 0.0f ? 1 : std::min(vocab, top_k);
  float sc[64];
  uint32_t id[64];
  if (qo_sample_topk(logits, seen, vocab, k, penalty, sc, id)) return 0xffffffffu;
  uint32_t selected = id[0];
  if (temperature > 0.0f && k > 1) {
    float total = 0.0f;
    const float maximum = sc[0];
    for (int j = 0; j < k; ++j) {
      sc[j] = float(std::exp(double((sc[j] - maximum) / temperature)));
      total += sc[j];
    }
    float retained = 0.0f;
    int count = 0;
    do {
      retained += sc[count];
      ++count;
    } while (count < k && retained < top_p * total);
    const float target = uniform * retained;
    float accumulated = 0.0f;
    selected = id[count - 1];
    for (int j = 0; j < count; ++j) {
      accumulated += sc[j];
      if (target < accumulated) {
        selected = id[j];
        break;
      }
    }
  }
  return selected;
}

}  // extern "C"
