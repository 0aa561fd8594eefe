// qnn_gguf.hip -- GGML block formats (Q8_0, Q4_K, Q5_K, Q6_K, Q3_K, Q2_K,
// IQ4_NL, IQ4_XS, Q2_0, IQ2_XXS, IQ2_S, IQ3_XXS, IQ3_S) for gfx950.
//
// Formats and decode rules: src/io/QuickNN.GGUF.Quantization.pas:136-253
// (GGUFValue); the matvec replaces op 65 (ggufvector.comp:34-52) and the GGUF
// gate/up SwiGLU op 67.
//
// Device layout.  Rows are tiled by 64 (one row per lane).  Each row is cut
// into 256-element units (a K-quant super-block, or 8 Q8_0 blocks).  The bytes
// of a unit are split into a "main" part whose size is a multiple of 16 bytes
// and up to two small side fields, each stored lane-interleaved:
//     main:  16 B at ((t*U + u)*C + c)*64 + r      (C chunks per unit)
//     side1: S1 B at ((t*U + u)*64 + r)            side2 likewise
//   Q4_K  (144 B): main 144 (C=9)
//   Q6_K  (210 B): main ql|qh|scales 208 (C=13), side1 d (2)
//   Q3_K  (110 B): main hmask|qs 96 (C=6), side1 scales (12), side2 d (2)
//   Q2_K   (84 B): main scales|qs 80 (C=5), side1 d|dmin (4)
//   Q8_0 (8x34 B): main 8x32 quants (C=16), side1 8 fp16 d (16)
//   Q5_K  (176 B): main 176 (C=11)
//   IQ4_XS (136 B): main quants 128 (C=8), side1 d|scales_h|scales_l (8)
//   IQ4_NL (8x18 B): main 8x16 quants (C=8), side1 8 fp16 d (16)
//   Q2_0  (4x18 B): main 4x16 quants (C=4), side1 4 fp16 d (8)
//   IQ2_XXS (66 B): main 64 (C=4), side1 d (2)
//   IQ2_S   (82 B): main qs|signs|qh|scales 80 (C=5), side1 d (2)
//   IQ3_XXS (98 B): main qs|signs+scales 96 (C=6), side1 d (2)
//   IQ3_S  (110 B): main qs|signs 96 (C=6), side1 qh|scales (12), side2 d (2)
// so every wave load is a 16-byte (or 12/8/4/2-byte) load by 64 consecutive
// lanes.  Bytes per weight are unchanged.
//
// Matvec.  The activation slice is quantised per 32 elements to 16-bit fixed
// point (x ~= s2 (256 q1 + q2), as in qnn_int4.hip) and each format's quants
// are unpacked into byte lanes for v_dot4_i32_i8; scale and min terms are
// applied once per sub-block:
//   Q4_K: sum = s2 * (d*sc * dot(q, X) - dmin*m * sum(X))       (sub-block 32)
//   Q2_K: sum = s2 * (d*sc * dot(q, X) - dmin*m * sum(X))       (sub-block 16)
//   Q6_K: sum = s2 * d*sc * (dot(q6, X) - 32 sum(X))            (q6 = q + 32)
//   Q3_K: sum = s2 * d*(sc-32) * (dot(q3, X) - 4 sum(X))        (q3 = q + 4)
//   Q8_0: sum = s2 * d * dot(q, X)
//   Q5_K: as Q4_K with 5-bit q (the fifth bit from qh)
//   IQ4_NL: sum = s2 * d * dot(v, X)                      (v = codebook byte)
//   IQ4_XS: sum = s2 * d*(ls-32) * dot(v, X)              (sub-block 32)
//   Q2_0:   sum = s2 * d * (dot(q, X) - sum(X))           (value d*(q-1))
//   IQ2/IQ3: sum = s2 * delta * dot(+-grid, X)   (per 32-group; IQ2_S per 16)
// where X = 256 q1 + q2 and every dot is exact integer arithmetic; the IQ4
// nibbles become their signed codebook bytes by a byte-permute lookup.  A
// Q2_0 byte holds four consecutive elements, so its activation slice is
// staged with each 16-element run transposed as a 4x4 byte matrix: word t
// then holds elements t, t+4, t+8, t+12, which is what one shift and mask of
// a quant word yields.  The IQ2/IQ3 grid codebook and a table of byte sign
// masks are copied into LDS by every workgroup; each 8 weights then take one
// grid lookup (two 4-byte entries for IQ3), one mask lookup, and the signs
// are applied to the grid bytes as (g ^ m) + (m & 0x01010101).
#include "qnn_int4_dev.h"  // buffer-load helpers (rsrc, ld128, ld32f) and the exchange
#include "qnn_iq_grids.h"

namespace qnn {
namespace {

__device__ __forceinline__ float silu_dev(float g) {  // tensor.comp:22, as GO_SWIGLU
  return g >= 20.0f ? g : (g <= -20.0f ? 0.0f : g / (1.0f + expf(-g)));
}
__device__ __forceinline__ float gelu_dev(float x) {  // tensor.comp:23 (tanh approximation), as GO_GEGLU
  return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}
// Weight loads: each weight byte is read once per launch, so they stream
// (non-temporal) and leave the L2 to the activations and the exchange
// (measured: Gemma-2 layer 43.2 -> 41.4 us).
typedef unsigned wl_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 wload(const uint4 *p) {
  const wl_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const wl_u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <class T> __device__ __forceinline__ T wload(const T *p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ uint32_t sel4u(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
// Exact binary16 -> binary32 (v_cvt_f32_f16; fp16 denormals are preserved).
__device__ __forceinline__ float half_f(uint32_t h) {
  const uint16_t b = uint16_t(h);
  _Float16 f;
  __builtin_memcpy(&f, &b, 2);
  return float(f);
}
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

__device__ __forceinline__ bool map_tile_slice(int b, int slices, int tiles, int &tile, int &slice) {
  const int xcd = b & 7, k = b >> 3;
  const int q = k / slices;
  tile = q * 8 + xcd;
  slice = k - q * slices;
  return tile < tiles;
}

// ---------------------------------------------------------------- format table
template <int ENC> struct Fmt;
template <> struct Fmt<QNN_WE_Q4_K> { static constexpr int C = 9, S1 = 0, S2 = 0; };
template <> struct Fmt<QNN_WE_Q6_K> { static constexpr int C = 13, S1 = 2, S2 = 0; };
template <> struct Fmt<QNN_WE_Q3_K> { static constexpr int C = 6, S1 = 12, S2 = 2; };
template <> struct Fmt<QNN_WE_Q2_K> { static constexpr int C = 5, S1 = 4, S2 = 0; };
template <> struct Fmt<QNN_WE_Q8_0> { static constexpr int C = 16, S1 = 16, S2 = 0; };
template <> struct Fmt<QNN_WE_Q5_K> { static constexpr int C = 11, S1 = 0, S2 = 0; };
template <> struct Fmt<QNN_WE_IQ4_XS> { static constexpr int C = 8, S1 = 8, S2 = 0; };
template <> struct Fmt<QNN_WE_IQ4_NL> { static constexpr int C = 8, S1 = 16, S2 = 0; };
template <> struct Fmt<QNN_WE_Q2_0> { static constexpr int C = 4, S1 = 8, S2 = 0; };
template <> struct Fmt<QNN_WE_IQ2_XXS> { static constexpr int C = 4, S1 = 2, S2 = 0; };
template <> struct Fmt<QNN_WE_IQ2_S> { static constexpr int C = 5, S1 = 2, S2 = 0; };
template <> struct Fmt<QNN_WE_IQ3_XXS> { static constexpr int C = 6, S1 = 2, S2 = 0; };
template <> struct Fmt<QNN_WE_IQ3_S> { static constexpr int C = 6, S1 = 12, S2 = 2; };

// ---------------------------------------------------------------- IQ2/IQ3 tables
// The codebooks (qnn_iq_grids.h), expanded at compile time into device memory,
// and byte sign masks: entry s of the 256 has byte i = 0xFF where bit i of s
// is set (IQ2_S, IQ3_S: 8 stored sign bits); entry s of the 128 is the mask of
// IQ2_SIGNS[s] (IQ2_XXS, IQ3_XXS: 7 stored bits, the eighth their parity).
constexpr uint64_t byte_mask(int s) {
  uint64_t m = 0;
  for (int i = 0; i < 8; ++i)
    if ((s >> i) & 1) m |= uint64_t(0xFF) << (8 * i);
  return m;
}
constexpr qnn_iq::Table<uint64_t, 256> sign_masks() {
  qnn_iq::Table<uint64_t, 256> t{};
  for (int s = 0; s < 256; ++s) t.v[s] = byte_mask(s);
  return t;
}
constexpr qnn_iq::Table<uint64_t, 128> sign_masks7() {
  qnn_iq::Table<uint64_t, 128> t{};
  const auto signs = qnn_iq::iq2_signs();
  for (int s = 0; s < 128; ++s) t.v[s] = byte_mask(signs.v[s]);
  return t;
}
__device__ const qnn_iq::Table<uint64_t, 256> kIQ2XXSGrid = qnn_iq::iq2xxs_grid();
__device__ const qnn_iq::Table<uint64_t, 1024> kIQ2SGrid = qnn_iq::iq2s_grid();
__device__ const qnn_iq::Table<uint32_t, 256> kIQ3XXSGrid = qnn_iq::iq3xxs_grid();
__device__ const qnn_iq::Table<uint32_t, 512> kIQ3SGrid = qnn_iq::iq3s_grid();
__device__ const qnn_iq::Table<uint8_t, 128> kIQ2Signs = qnn_iq::iq2_signs();
__device__ const qnn_iq::Table<uint64_t, 256> kSignMasks = sign_masks();
__device__ const qnn_iq::Table<uint64_t, 128> kSignMasks7 = sign_masks7();

template <int ENC> constexpr bool kIsIQ =
    ENC == QNN_WE_IQ2_XXS || ENC == QNN_WE_IQ2_S || ENC == QNN_WE_IQ3_XXS || ENC == QNN_WE_IQ3_S;
// Bytes of the format's codebook (0 for the other formats).
template <int ENC> constexpr int kIQGridBytes = ENC == QNN_WE_IQ2_XXS ? 2048 : ENC == QNN_WE_IQ2_S ? 8192
                                                : ENC == QNN_WE_IQ3_XXS ? 1024 : ENC == QNN_WE_IQ3_S ? 2048 : 0;
template <int ENC> __device__ __forceinline__ const uint4 *iq_grid_src() {
  if constexpr (ENC == QNN_WE_IQ2_XXS) return reinterpret_cast<const uint4 *>(kIQ2XXSGrid.v);
  if constexpr (ENC == QNN_WE_IQ2_S) return reinterpret_cast<const uint4 *>(kIQ2SGrid.v);
  if constexpr (ENC == QNN_WE_IQ3_XXS) return reinterpret_cast<const uint4 *>(kIQ3XXSGrid.v);
  return reinterpret_cast<const uint4 *>(kIQ3SGrid.v);
}
// 16-byte pieces of the sign-mask table a format uses.
template <int ENC> constexpr int kIQMaskU4 = (ENC == QNN_WE_IQ2_XXS || ENC == QNN_WE_IQ3_XXS) ? 64 : 128;
template <int ENC> __device__ __forceinline__ const uint4 *iq_mask_src() {
  if constexpr (kIQMaskU4<ENC> == 64) return reinterpret_cast<const uint4 *>(kSignMasks7.v);
  return reinterpret_cast<const uint4 *>(kSignMasks.v);
}
__device__ __forceinline__ uint32_t apply_sign(uint32_t g, uint32_t m) { return (g ^ m) + (m & 0x01010101u); }

// IQ4_NL_VALUES (src/io/QuickNN.GGUF.Quantization.pas:34) as signed bytes,
// four per word: the codebook of IQ4_NL and IQ4_XS.
constexpr uint32_t kIQ4W0 = 0xBFAD9881u;  // -127, -104,  -83,  -65
constexpr uint32_t kIQ4W1 = 0xF6EADDCFu;  //  -49,  -35,  -22,  -10
constexpr uint32_t kIQ4W2 = 0x26190D01u;  //    1,   13,   25,   38
constexpr uint32_t kIQ4W3 = 0x71594535u;  //   53,   69,   89,  113
__host__ __device__ constexpr int iq4_value(int q) {
  return int(int8_t(((q < 4 ? kIQ4W0 : q < 8 ? kIQ4W1 : q < 12 ? kIQ4W2 : kIQ4W3) >> (8 * (q & 3))) & 255u));
}
static_assert(iq4_value(0) == -127 && iq4_value(1) == -104 && iq4_value(2) == -83 && iq4_value(3) == -65 &&
                  iq4_value(4) == -49 && iq4_value(5) == -35 && iq4_value(6) == -22 && iq4_value(7) == -10 &&
                  iq4_value(8) == 1 && iq4_value(9) == 13 && iq4_value(10) == 25 && iq4_value(11) == 38 &&
                  iq4_value(12) == 53 && iq4_value(13) == 69 && iq4_value(14) == 89 && iq4_value(15) == 113,
              "IQ4_NL_VALUES");
// Four nibbles (one per byte, 0-15) -> their four codebook bytes: two byte
// permutes over the 8-entry halves, then a per-byte select on bit 3.
__device__ __forceinline__ uint32_t iq4_bytes(uint32_t nib) {
  const uint32_t sel = nib & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(kIQ4W1, kIQ4W0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(kIQ4W3, kIQ4W2, sel);
  const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}

// Lane t (0-3) of each quad of lanes receives byte t of the quad's four
// words, the word of lane s in byte s: a 4x4 byte transpose.
__device__ __forceinline__ uint32_t quad_transpose(uint32_t v, int t) {
  const uint32_t v0 = dev::dpp<0x00>(v), v1 = dev::dpp<0x55>(v), v2 = dev::dpp<0xAA>(v), v3 = dev::dpp<0xFF>(v);
  const uint32_t lo = __builtin_amdgcn_perm(v1, v0, uint32_t(t) | (uint32_t(t + 4) << 8) | 0x0C0C0000u);
  const uint32_t hi = __builtin_amdgcn_perm(v3, v2, 0x0C0Cu | (uint32_t(t) << 16) | (uint32_t(t + 4) << 24));
  return lo | hi;
}

struct Planes {
  const uint8_t *main;
  const uint8_t *side1;
  const uint8_t *side2;
};

__device__ __forceinline__ Planes planes_of(const GGLayout &l, const void *w) {
  const uint8_t *b = static_cast<const uint8_t *>(w);
  Planes p;
  p.main = b;
  p.side1 = b + l.side1_off;
  p.side2 = b + l.side2_off;
  return p;
}

// Original byte `o` (0 <= o < unit bytes) of unit (t, u) row r, through the
// plane mapping.  Used by the repack (inverse) and the bit-exact dequant.
__device__ __forceinline__ void plane_addr(int enc, const GGLayout &l, int t, int u, int r, int o, int &plane,
                                           size_t &off) {
  const size_t tu = size_t(t) * l.units + u;
  auto main_at = [&](int m) { plane = 0; off = ((tu * l.main_chunks + (m >> 4)) * 64 + r) * 16 + (m & 15); };
  auto s1_at = [&](int m) { plane = 1; off = (tu * 64 + r) * l.side1_bytes + m; };
  auto s2_at = [&](int m) { plane = 2; off = (tu * 64 + r) * l.side2_bytes + m; };
  switch (enc) {
    case QNN_WE_Q4_K: main_at(o); break;
    case QNN_WE_Q6_K: if (o < 208) main_at(o); else s1_at(o - 208); break;
    case QNN_WE_Q3_K: if (o < 96) main_at(o); else if (o < 108) s1_at(o - 96); else s2_at(o - 108); break;
    case QNN_WE_Q2_K: if (o < 80) main_at(o); else s1_at(o - 80); break;
    case QNN_WE_Q5_K: main_at(o); break;
    case QNN_WE_IQ4_XS: if (o < 8) s1_at(o); else main_at(o - 8); break;
    case QNN_WE_IQ2_XXS: case QNN_WE_IQ2_S: case QNN_WE_IQ3_XXS: if (o < 2) s1_at(o); else main_at(o - 2); break;
    case QNN_WE_IQ3_S:  // d | qs 64 | qh 8 | signs 32 | scales 4
      if (o < 2) s2_at(o);
      else if (o < 66) main_at(o - 2);
      else if (o < 74) s1_at(o - 66);
      else if (o < 106) main_at(o - 10);
      else s1_at(o - 98);
      break;
    case QNN_WE_IQ4_NL:
    case QNN_WE_Q2_0: {  // unit of 8 (4) blocks: block k = o / 18, byte j = o % 18: d at j < 2, quants after
      const int k = o / 18, j = o % 18;
      if (j < 2) s1_at(2 * k + j); else main_at(16 * k + j - 2);
      break;
    }
    default: {  // Q8_0 unit: block k = o / 34, byte j = o % 34: d at j < 2, quants after
      const int k = o / 34, j = o % 34;
      if (j < 2) s1_at(2 * k + j); else main_at(32 * k + j - 2);
    }
  }
}

__device__ __forceinline__ uint32_t fetch(int enc, const GGLayout &l, const Planes &p, int t, int u, int r, int o) {
  int plane;
  size_t off;
  plane_addr(enc, l, t, u, r, o, plane, off);
  return plane == 0 ? p.main[off] : (plane == 1 ? p.side1[off] : p.side2[off]);
}

// GGUFValue (src/io/QuickNN.GGUF.Quantization.pas:136-253) over the tiled
// copy: element i of unit (t, u), row r.  Same arithmetic, so the same bits.
__device__ float gguf_value_tiled(int enc, const GGLayout &l, const Planes &p, int t, int u, int r, int i) {
  auto B = [&](int o) { return fetch(enc, l, p, t, u, r, o); };
  auto H = [&](int o) { return half_f(B(o) | (B(o + 1) << 8)); };
  auto SB = [](uint32_t v) { return v >= 128 ? int(v) - 256 : int(v); };
  switch (enc) {
    case QNN_WE_Q8_0: {
      const int k = i / 32, j = i % 32;
      return H(34 * k) * float(SB(B(34 * k + 2 + j)));
    }
    case QNN_WE_Q2_K: {
      const int group = i / 16;
      const int q = int((B(16 + (i / 128) * 32 + i % 32) >> (((i % 128) / 32) * 2)) & 3);
      return (H(80) * float(B(group) & 15)) * float(q) - H(82) * float(B(group) >> 4);
    }
    case QNN_WE_Q4_K:
    case QNN_WE_Q5_K: {  // Q5_K: quants at 48, the fifth bit from byte 16 + i % 32
      const int group = i / 32;
      int scale, minimum;
      if (group < 4) {
        scale = int(B(4 + group) & 63);
        minimum = int(B(8 + group) & 63);
      } else {
        scale = int((B(8 + group) & 15) | ((B(group) >> 6) << 4));
        minimum = int((B(8 + group) >> 4) | ((B(4 + group) >> 6) << 4));
      }
      int q = int((B((enc == QNN_WE_Q5_K ? 48 : 16) + (i / 64) * 32 + i % 32) >> ((group & 1) * 4)) & 15);
      if (enc == QNN_WE_Q5_K) q |= int((B(16 + i % 32) >> group) & 1u) << 4;
      return (H(0) * float(scale)) * float(q) - H(2) * float(minimum);
    }
    case QNN_WE_IQ4_NL: {
      const int k = i / 32, j = i % 32;
      const int q = int((B(18 * k + 2 + j % 16) >> ((j / 16) * 4)) & 15);
      return H(18 * k) * float(iq4_value(q));
    }
    case QNN_WE_IQ3_XXS: {  // GGUF.Quantization.pas:148-157
      const int group = i / 32;
      const uint32_t bits = B(66 + group * 4) | (B(67 + group * 4) << 8) | (B(68 + group * 4) << 16) |
                            (B(69 + group * 4) << 24);
      const uint32_t signs = kIQ2Signs.v[(bits >> (7 * ((i % 32) / 8))) & 127];
      int q = int((kIQ3XXSGrid.v[B(2 + i / 4)] >> ((i % 4) * 8)) & 255);
      if (signs & (1u << (i % 8))) q = -q;
      return (H(0) * (0.5f + float(bits >> 28)) * 0.5f) * float(q);
    }
    case QNN_WE_IQ2_XXS:
    case QNN_WE_IQ2_S: {  // :158-179
      const int group = i / 32, lane = (i % 32) / 8;
      uint64_t grid;
      uint32_t signs;
      float delta;
      if (enc == QNN_WE_IQ2_XXS) {
        const uint32_t bits = B(6 + group * 8) | (B(7 + group * 8) << 8) | (B(8 + group * 8) << 16) |
                              (B(9 + group * 8) << 24);
        grid = kIQ2XXSGrid.v[B(2 + group * 8 + lane)];
        signs = kIQ2Signs.v[(bits >> (7 * lane)) & 127];
        delta = H(0) * (0.5f + float(bits >> 28)) * 0.25f;
      } else {
        grid = kIQ2SGrid.v[B(2 + group * 4 + lane) | (((B(66 + group) >> (lane * 2)) & 3) << 8)];
        signs = B(34 + i / 8);
        delta = H(0) * (0.5f + float((B(74 + group) >> (((i % 32) / 16) * 4)) & 15)) * 0.25f;
      }
      int q = int((grid >> ((i % 8) * 8)) & 255);
      if (signs & (1u << (i % 8))) q = -q;
      return delta * float(q);
    }
    case QNN_WE_IQ3_S: {  // :242-251
      const int group = i / 32;
      const uint32_t gi = B(2 + i / 4) | (((B(66 + group) >> ((i % 32) / 4)) & 1) << 8);
      int q = int((kIQ3SGrid.v[gi] >> ((i % 4) * 8)) & 255);
      if (B(74 + i / 8) & (1u << (i % 8))) q = -q;
      const int scale = 1 + 2 * int((B(106 + group / 2) >> ((group % 2) * 4)) & 15);
      return (H(0) * float(scale)) * float(q);
    }
    case QNN_WE_Q2_0: {  // GGUF.Quantization.pas:146-147
      const int k = i / 64, j = i % 64;
      const int q = int((B(18 * k + 2 + j / 4) >> ((j % 4) * 2)) & 3);
      return H(18 * k) * float(q - 1);
    }
    case QNN_WE_IQ4_XS: {
      const int group = i / 32;
      const int scale = int(((B(4 + group / 2) >> ((group % 2) * 4)) & 15) |
                            ((((B(2) | (B(3) << 8)) >> (group * 2)) & 3) << 4));
      const int q = int((B(8 + group * 16 + i % 16) >> (((i % 32) / 16) * 4)) & 15);
      return (H(0) * float(scale - 32)) * float(iq4_value(q));
    }
    case QNN_WE_Q6_K: {
      const int part = i / 128, quarter = (i % 128) / 32, lane = i % 32;
      const int q = int(((B(part * 64 + (quarter & 1) * 32 + lane) >> ((quarter / 2) * 4)) & 15) |
                        (((B(128 + part * 32 + lane) >> (quarter * 2)) & 3) << 4));
      const int scale = SB(B(192 + i / 16));
      return (H(208) * float(scale)) * float(q - 32);
    }
    default: {  // Q3_K
      const int group = i / 16;
      const int scale = int(((B(96 + group % 8) >> ((group / 8) * 4)) & 15) |
                            (((B(104 + group % 4) >> ((group / 4) * 2)) & 3) << 4));
      int q = int((B(32 + (i / 128) * 32 + i % 32) >> (((i % 128) / 32) * 2)) & 3);
      if ((B(i % 32) & (1u << (i / 32))) == 0) q -= 4;
      return (H(108) * float(scale - 32)) * float(q);
    }
  }
}

// ---------------------------------------------------------------- repack / dequant kernels
__global__ void k_gguf_repack(const uint8_t *__restrict__ src, GGLayout l, uint8_t *__restrict__ dst) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = size_t(l.tiles) * l.units * 64;
  if (idx >= total) return;
  const int r = int(idx & 63);
  const int u = int((idx >> 6) % l.units);
  const int t = int(idx / (size_t(l.units) * 64));
  const int row = t * 64 + r;
  const int ub = l.unit_bytes;
  const size_t row_bytes = size_t(l.src_row_bytes);
  for (int o = 0; o < ub; ++o) {
    uint8_t v = 0;
    if (row < l.rows) {
      const size_t so = size_t(u) * ub + o;  // Q8_0 / IQ4_NL / Q2_0 units past the row end are zero blocks (d = 0)
      if (so < row_bytes) v = src[size_t(row) * row_bytes + so];
    }
    int plane;
    size_t off;
    plane_addr(l.enc, l, t, u, r, o, plane, off);
    dst[(plane == 0 ? 0 : (plane == 1 ? l.side1_off : l.side2_off)) + off] = v;
  }
}

__global__ void k_gguf_dequant(GGLayout l, const uint8_t *__restrict__ w, float *__restrict__ out) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = size_t(l.rows) * l.cols;
  if (idx >= total) return;
  const int row = int(idx / l.cols), k = int(idx % l.cols);
  const Planes p = planes_of(l, w);
  out[idx] = gguf_value_tiled(l.enc, l, p, row / 64, k / 256, row & 63, k % 256);
}

// fp16 copy for the multi-row GEMM (k_h16_gemm).  Row exponents: one
// workgroup per row of the copy, the largest |GGUFValue| of the row (rows past
// the weight give 0).
__global__ __launch_bounds__(256) void k_gguf_rowexp(GGLayout l, const uint8_t *__restrict__ w, int *__restrict__ ew) {
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  float amax = 0.0f;
  if (row < l.rows) {
    const Planes p = planes_of(l, w);
    for (int k = tid; k < l.cols; k += 256)
      amax = fmaxf(amax, fabsf(gguf_value_tiled(l.enc, l, p, row / 64, k / 256, row & 63, k % 256)));
  }
  amax = dev::wave_max_xor(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  if (tid == 0) ew[row] = range_exp(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
}
// The values: piece (n32, ks, lane) = 8 halfs RNE(W[n][k] * 2^-ew[n]) for
// n = n32*32 + lane % 32, k = ks*16 + 8*(lane / 32) + 0..7 (the B operand
// fragments of v_mfma_f32_32x32x16_f16); rows past N and columns past K are
// zero.
__global__ __launch_bounds__(256) void k_gguf_expand_h16(GGLayout l, const uint8_t *__restrict__ w,
                                                         const int *__restrict__ ew, int ksteps, size_t pieces,
                                                         uint4 *__restrict__ out) {
  const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= pieces) return;
  const int lane = int(idx & 63);
  const size_t nk = idx >> 6;
  const int ks = int(nk % ksteps), n32 = int(nk / ksteps);
  const int n = n32 * 32 + (lane & 31), k0 = ks * 16 + 8 * (lane >> 5);
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (n < l.rows && k0 < l.cols) {  // cols is a multiple of 32: all 8 columns are in the row
    const Planes p = planes_of(l, w);
    const float sc = ldexpf(1.0f, -ew[n]);
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = gguf_value_tiled(l.enc, l, p, n / 64, (k0 + i) / 256, n & 63, (k0 + i) % 256) * sc;
    v = make_uint4(pack_h2(f[0], f[1]), pack_h2(f[2], f[3]), pack_h2(f[4], f[5]), pack_h2(f[6], f[7]));
  }
  out[idx] = v;
}

// Gather (Context.Implementation.inc:1228-1267, tensor.comp:245-251 with a
// GGUF weight): out[r][k] = value of row ids[r] (raw token bits) column k, or 0
// for ids at or past the vocabulary.
__global__ void k_gguf_gather(GGLayout l, const uint8_t *__restrict__ w, const unsigned *__restrict__ ids,
                              float *__restrict__ out, int rows, int vocab) {
  const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= size_t(rows) * l.cols) return;
  const int r = int(idx / l.cols), k = int(idx % l.cols);
  const unsigned token = ids[r];
  if (token >= unsigned(vocab)) {
    out[idx] = 0.0f;
    return;
  }
  const Planes p = planes_of(l, w);
  out[idx] = gguf_value_tiled(l.enc, l, p, int(token / 64), k / 256, int(token & 63), k % 256);
}

// ---------------------------------------------------------------- matvec
// Fixed-point activation slice of one token, in LDS: per 32-group 8 words of
// q1 and q2 bytes (element order), s2, and the sums of X = 256 q1 + q2 over
// the group and over each 16-element half.
template <int NG>
struct XSlice {
  uint32_t h[NG][8];
  uint32_t l[NG][8];
  float s2[NG];
  int sum32[NG];
  int sum16[NG][2];
};

// Exact integer dot of four quant bytes with four activation bytes (q1, q2).
__device__ __forceinline__ int xdot(uint32_t q, uint32_t xh, uint32_t xl, int &acc_h, int &acc_l) {
  acc_h = dot4(q, xh, acc_h);
  acc_l = dot4(q, xl, acc_l);
  return 0;
}

template <int NG>
__device__ __forceinline__ int combine(int ah, int al) { return (ah << 8) + al; }

// Unit dot products.  `mw` = main chunks (registers), s1/s2 side words.
// g0: first 32-group of this unit within the LDS slice.
template <int NG>
__device__ float unit_q8_0(const uint4 *mw, uint4 s1, const XSlice<NG> &xs, int g0) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {  // block k: quants in chunks 2k, 2k+1
    int ah = 0, al = 0;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) xdot(sel4u(mw[2 * k + c], j), xs.h[g0 + k][4 * c + j], xs.l[g0 + k][4 * c + j], ah, al);
    const uint32_t dw = sel4u(s1, k >> 1);
    const float d = half_f((k & 1) ? (dw >> 16) : (dw & 0xFFFFu));
    acc = fmaf(float(combine<NG>(ah, al)), d * xs.s2[g0 + k], acc);
  }
  return acc;
}

template <int NG>
__device__ float unit_q4_k(const uint4 *mw, const XSlice<NG> &xs, int g0) {
  const uint4 hd = mw[0];
  const float d = half_f(hd.x & 0xFFFFu), dmin = half_f(hd.x >> 16);
  const uint32_t s0 = hd.y, s4 = hd.z, s8 = hd.w;  // scale bytes 0-3, 4-7, 8-11
  auto byte = [&](int b) -> uint32_t {
    const uint32_t w = b < 4 ? s0 : (b < 8 ? s4 : s8);
    return (w >> (8 * (b & 3))) & 255u;
  };
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int sc, m;
    if (j < 4) {
      sc = int(byte(j) & 63);
      m = int(byte(4 + j) & 63);
    } else {
      sc = int((byte(4 + j) & 15) | ((byte(j - 4) >> 6) << 4));
      m = int((byte(4 + j) >> 4) | ((byte(j) >> 6) << 4));
    }
    int ah = 0, al = 0;
    // quants of sub-block j: bytes (j/2)*32 .. +31 of the quant area (chunks 1 + 2*(j/2), +1)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t qd = sel4u(mw[1 + 2 * (j >> 1) + c], w);
        const uint32_t q = (j & 1) ? ((qd >> 4) & 0x0F0F0F0Fu) : (qd & 0x0F0F0F0Fu);
        xdot(q, xs.h[g0 + j][4 * c + w], xs.l[g0 + j][4 * c + w], ah, al);
      }
    const float isum = float(combine<NG>(ah, al));
    acc = fmaf(xs.s2[g0 + j], (d * float(sc)) * isum - (dmin * float(m)) * float(xs.sum32[g0 + j]), acc);
  }
  return acc;
}

template <int NG>
__device__ float unit_q6_k(const uint4 *mw, uint32_t side, const XSlice<NG> &xs, int g0) {
  const float d = half_f(side & 0xFFFFu);
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // elements 128p + 32q .. +31 = 32-group 4p + q
      const int g = 4 * p + q;
      int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int qlw = p * 16 + (q & 1) * 8 + k;  // ql dword (chunks 0-7)
        const int qhw = 32 + p * 8 + k;            // qh dword (chunks 8-11)
        const uint32_t ql = sel4u(mw[qlw >> 2], qlw & 3), qh = sel4u(mw[qhw >> 2], qhw & 3);
        const uint32_t v = ((ql >> ((q >> 1) * 4)) & 0x0F0F0F0Fu) | (((qh >> (2 * q)) & 0x03030303u) << 4);
        if (k < 4) xdot(v, xs.h[g0 + g][k], xs.l[g0 + g][k], ah0, al0);
        else xdot(v, xs.h[g0 + g][k], xs.l[g0 + g][k], ah1, al1);
      }
      const uint4 scw = mw[12];
      const int sb0 = 2 * g, sb1 = 2 * g + 1;  // 16-element sub-blocks
      const int sc0 = int(int8_t((sel4u(scw, sb0 >> 2) >> (8 * (sb0 & 3))) & 255u));
      const int sc1 = int(int8_t((sel4u(scw, sb1 >> 2) >> (8 * (sb1 & 3))) & 255u));
      const int i0 = combine<NG>(ah0, al0) - 32 * xs.sum16[g0 + g][0];
      const int i1 = combine<NG>(ah1, al1) - 32 * xs.sum16[g0 + g][1];
      acc = fmaf(xs.s2[g0 + g] * d, float(sc0) * float(i0) + float(sc1) * float(i1), acc);
    }
  return acc;
}

template <int NG>
__device__ float unit_q3_k(const uint4 *mw, uint4 s1, uint32_t s2w, const XSlice<NG> &xs, int g0) {
  const float d = half_f(s2w & 0xFFFFu);
  auto sbyte = [&](int b) -> uint32_t { return (sel4u(s1, b >> 2) >> (8 * (b & 3))) & 255u; };
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = 4 * p + q;
      int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int qsw = 8 + p * 8 + k;  // qs dword (chunks 2-5)
        const int hmw = k;              // hmask dword (chunks 0-1)
        const uint32_t qs = sel4u(mw[qsw >> 2], qsw & 3), hm = sel4u(mw[hmw >> 2], hmw & 3);
        const uint32_t v = ((qs >> (2 * q)) & 0x03030303u) | (((hm >> (4 * p + q)) & 0x01010101u) << 2);
        if (k < 4) xdot(v, xs.h[g0 + g][k], xs.l[g0 + g][k], ah0, al0);
        else xdot(v, xs.h[g0 + g][k], xs.l[g0 + g][k], ah1, al1);
      }
      int sc[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int sb = 2 * g + hh;
        sc[hh] = int(((sbyte(sb % 8) >> ((sb / 8) * 4)) & 15) | (((sbyte(8 + sb % 4) >> ((sb / 4) * 2)) & 3) << 4)) - 32;
      }
      const int i0 = combine<NG>(ah0, al0) - 4 * xs.sum16[g0 + g][0];
      const int i1 = combine<NG>(ah1, al1) - 4 * xs.sum16[g0 + g][1];
      acc = fmaf(xs.s2[g0 + g] * d, float(sc[0]) * float(i0) + float(sc[1]) * float(i1), acc);
    }
  return acc;
}

template <int NG>
__device__ float unit_q2_k(const uint4 *mw, uint32_t side, const XSlice<NG> &xs, int g0) {
  const float d = half_f(side & 0xFFFFu), dmin = half_f(side >> 16);
  float acc = 0.0f;
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = 4 * p + q;
      int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int qsw = 4 + p * 8 + k;  // qs dword (chunks 1-4)
        const uint32_t qs = sel4u(mw[qsw >> 2], qsw & 3);
        const uint32_t v = (qs >> (2 * q)) & 0x03030303u;
        if (k < 4) xdot(v, xs.h[g0 + g][k], xs.l[g0 + g][k], ah0, al0);
        else xdot(v, xs.h[g0 + g][k], xs.l[g0 + g][k], ah1, al1);
      }
      float part = 0.0f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int sb = 2 * g + hh;
        const uint32_t sm = (sel4u(mw[0], sb >> 2) >> (8 * (sb & 3))) & 255u;
        const int isum = hh ? combine<NG>(ah1, al1) : combine<NG>(ah0, al0);
        part += (d * float(sm & 15)) * float(isum) - (dmin * float(sm >> 4)) * float(xs.sum16[g0 + g][hh]);
      }
      acc = fmaf(xs.s2[g0 + g], part, acc);
    }
  return acc;
}

template <int NG>
__device__ float unit_q5_k(const uint4 *mw, const XSlice<NG> &xs, int g0) {
  const uint4 hd = mw[0];
  const float d = half_f(hd.x & 0xFFFFu), dmin = half_f(hd.x >> 16);
  const uint32_t s0 = hd.y, s4 = hd.z, s8 = hd.w;
  auto byte = [&](int b) -> uint32_t {
    const uint32_t w = b < 4 ? s0 : (b < 8 ? s4 : s8);
    return (w >> (8 * (b & 3))) & 255u;
  };
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int sc, m;
    if (j < 4) {
      sc = int(byte(j) & 63);
      m = int(byte(4 + j) & 63);
    } else {
      sc = int((byte(4 + j) & 15) | ((byte(j - 4) >> 6) << 4));
      m = int((byte(4 + j) >> 4) | ((byte(j) >> 6) << 4));
    }
    int ah = 0, al = 0;
    // sub-block j: low nibbles at bytes 48 + (j/2)*32 (chunks 3 + 2*(j/2), +1),
    // fifth bits at bytes 16..47 (chunks 1, 2), bit j
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t qd = sel4u(mw[3 + 2 * (j >> 1) + c], w), hb = sel4u(mw[1 + c], w);
        const uint32_t q = (((j & 1) ? (qd >> 4) : qd) & 0x0F0F0F0Fu) | (((hb >> j) & 0x01010101u) << 4);
        xdot(q, xs.h[g0 + j][4 * c + w], xs.l[g0 + j][4 * c + w], ah, al);
      }
    const float isum = float(combine<NG>(ah, al));
    acc = fmaf(xs.s2[g0 + j], (d * float(sc)) * isum - (dmin * float(m)) * float(xs.sum32[g0 + j]), acc);
  }
  return acc;
}

// The integer dot of one 32-group of IQ4 nibbles (16 bytes: low nibbles are
// elements 0-15, high nibbles 16-31) with the group's activation planes.
template <int NG>
__device__ __forceinline__ int iq4_group_dot(const uint4 &qs, const XSlice<NG> &xs, int g) {
  int ah = 0, al = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const uint32_t qd = sel4u(qs, w & 3);
    const uint32_t v = iq4_bytes(((w < 4) ? qd : (qd >> 4)) & 0x0F0F0F0Fu);
    xdot(v, xs.h[g][w], xs.l[g][w], ah, al);
  }
  return combine<NG>(ah, al);
}

template <int NG>
__device__ float unit_iq4_nl(const uint4 *mw, uint4 s1, const XSlice<NG> &xs, int g0) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {  // block k: quants in chunk k, d in side half k
    const uint32_t dw = sel4u(s1, k >> 1);
    const float d = half_f((k & 1) ? (dw >> 16) : (dw & 0xFFFFu));
    acc = fmaf(float(iq4_group_dot<NG>(mw[k], xs, g0 + k)), d * xs.s2[g0 + k], acc);
  }
  return acc;
}

// Q2_0: block k (64 elements, groups g0 + 2k and g0 + 2k + 1) in chunk k, its
// d in side half k.  Quant word w of the chunk holds elements 16w..16w+15,
// four per byte; shift 2t and mask give elements 16w + t + {0, 4, 8, 12},
// the order of the transposed activation word 4(w & 1) + t.
template <int NG>
__device__ float unit_q2_0(const uint4 *mw, uint4 s1, const XSlice<NG> &xs, int g0) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t dw = sel4u(s1, k >> 1);
    const float d = half_f((k & 1) ? (dw >> 16) : (dw & 0xFFFFu));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = g0 + 2 * k + h;
      int ah = 0, al = 0;
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const uint32_t qw = sel4u(mw[k], 2 * h + w);
#pragma unroll
        for (int t = 0; t < 4; ++t) xdot((qw >> (2 * t)) & 0x03030303u, xs.h[g][4 * w + t], xs.l[g][4 * w + t], ah, al);
      }
      acc = fmaf(float(combine<NG>(ah, al) - xs.sum32[g]), d * xs.s2[g], acc);
    }
  }
  return acc;
}

// IQ2/IQ3 units.  `grid` and `mask` point at the LDS copies of the codebook
// and of the sign masks (indexed by the 7 stored bits for IQ2_XXS and
// IQ3_XXS, by the sign byte for IQ2_S and IQ3_S).  8 weights (lane L of a 32-group) are one 8-byte
// grid entry (IQ2) or two 4-byte entries (IQ3) against activation words 2L
// and 2L + 1 of the group.
template <int NG>
__device__ __forceinline__ void iq_dot8(uint64_t grid, uint64_t mask, const XSlice<NG> &xs, int g, int L, int &ah,
                                        int &al) {
  xdot(apply_sign(uint32_t(grid), uint32_t(mask)), xs.h[g][2 * L], xs.l[g][2 * L], ah, al);
  xdot(apply_sign(uint32_t(grid >> 32), uint32_t(mask >> 32)), xs.h[g][2 * L + 1], xs.l[g][2 * L + 1], ah, al);
}

template <int NG>
__device__ float unit_iq2_xxs(const uint4 *mw, uint32_t dh, const XSlice<NG> &xs, int g0, const uint64_t *grid,
                              const uint64_t *mask) {
  const float d = half_f(dh);
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {  // group g: 4 grid indices, then 4 x 7 sign bits and a 4-bit scale
    const uint32_t idx = sel4u(mw[g >> 1], 2 * (g & 1)), bits = sel4u(mw[g >> 1], 2 * (g & 1) + 1);
    int ah = 0, al = 0;
#pragma unroll
    for (int L = 0; L < 4; ++L)
      iq_dot8<NG>(grid[(idx >> (8 * L)) & 255u], mask[(bits >> (7 * L)) & 127u], xs, g0 + g, L, ah, al);
    const float delta = d * (0.5f + float(bits >> 28)) * 0.25f;
    acc = fmaf(float(combine<NG>(ah, al)), delta * xs.s2[g0 + g], acc);
  }
  return acc;
}

template <int NG>
__device__ float unit_iq2_s(const uint4 *mw, uint32_t dh, const XSlice<NG> &xs, int g0, const uint64_t *grid,
                            const uint64_t *mask) {
  // main: qs 0-31 (chunks 0-1), signs 32-63 (chunks 2-3), qh 64-71 and scales 72-79 (chunk 4)
  const float d = half_f(dh);
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t qs = sel4u(mw[g >> 2], g & 3), sg = sel4u(mw[2 + (g >> 2)], g & 3);
    const uint32_t qh = (sel4u(mw[4], g >> 2) >> (8 * (g & 3))) & 255u;
    const uint32_t sc = (sel4u(mw[4], 2 + (g >> 2)) >> (8 * (g & 3))) & 255u;
    int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      const uint32_t gi = ((qs >> (8 * L)) & 255u) | (((qh >> (2 * L)) & 3u) << 8);
      if (L < 2) iq_dot8<NG>(grid[gi], mask[(sg >> (8 * L)) & 255u], xs, g0 + g, L, ah0, al0);
      else iq_dot8<NG>(grid[gi], mask[(sg >> (8 * L)) & 255u], xs, g0 + g, L, ah1, al1);
    }
    const float d0 = d * (0.5f + float(sc & 15u)) * 0.25f, d1 = d * (0.5f + float(sc >> 4)) * 0.25f;
    acc = fmaf(float(combine<NG>(ah0, al0)), d0 * xs.s2[g0 + g], acc);
    acc = fmaf(float(combine<NG>(ah1, al1)), d1 * xs.s2[g0 + g], acc);
  }
  return acc;
}

template <int NG>
__device__ float unit_iq3_xxs(const uint4 *mw, uint32_t dh, const XSlice<NG> &xs, int g0, const uint32_t *grid,
                              const uint64_t *mask) {
  // main: 64 grid indices (chunks 0-3, 8 per group), then 8 words of 4 x 7 sign bits and a 4-bit scale
  const float d = half_f(dh);
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t i0 = sel4u(mw[g >> 1], 2 * (g & 1)), i1 = sel4u(mw[g >> 1], 2 * (g & 1) + 1);
    const uint32_t bits = sel4u(mw[4 + (g >> 2)], g & 3);
    int ah = 0, al = 0;
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      const uint32_t iw = L < 2 ? i0 : i1;
      const uint32_t a = grid[(iw >> (16 * (L & 1))) & 255u], b = grid[(iw >> (16 * (L & 1) + 8)) & 255u];
      iq_dot8<NG>(uint64_t(a) | (uint64_t(b) << 32), mask[(bits >> (7 * L)) & 127u], xs, g0 + g, L, ah, al);
    }
    const float delta = d * (0.5f + float(bits >> 28)) * 0.5f;
    acc = fmaf(float(combine<NG>(ah, al)), delta * xs.s2[g0 + g], acc);
  }
  return acc;
}

template <int NG>
__device__ float unit_iq3_s(const uint4 *mw, uint4 s1, uint32_t dh, const XSlice<NG> &xs, int g0,
                            const uint32_t *grid, const uint64_t *mask) {
  // main: 64 low grid-index bytes (chunks 0-3), 32 sign bytes (chunks 4-5); side1: qh 8 | scales 4
  const float d = half_f(dh);
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const uint32_t i0 = sel4u(mw[g >> 1], 2 * (g & 1)), i1 = sel4u(mw[g >> 1], 2 * (g & 1) + 1);
    const uint32_t sg = sel4u(mw[4 + (g >> 2)], g & 3);
    const uint32_t qh = (sel4u(s1, g >> 2) >> (8 * (g & 3))) & 255u;
    const uint32_t sc = (s1.z >> (4 * g)) & 15u;
    int ah = 0, al = 0;
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      const uint32_t iw = L < 2 ? i0 : i1;
      const int j = 2 * L;  // 4-element pieces j, j + 1 of the group
      const uint32_t a = grid[((iw >> (16 * (L & 1))) & 255u) | (((qh >> j) & 1u) << 8)];
      const uint32_t b = grid[((iw >> (16 * (L & 1) + 8)) & 255u) | (((qh >> (j + 1)) & 1u) << 8)];
      iq_dot8<NG>(uint64_t(a) | (uint64_t(b) << 32), mask[(sg >> (8 * L)) & 255u], xs, g0 + g, L, ah, al);
    }
    acc = fmaf(float(combine<NG>(ah, al)), (d * float(1u + 2u * sc)) * xs.s2[g0 + g], acc);
  }
  return acc;
}

template <int NG>
__device__ float unit_iq4_xs(const uint4 *mw, uint4 s1, const XSlice<NG> &xs, int g0) {
  // side: bytes 0-1 d, 2-3 scales_h, 4-7 scales_l
  const float d = half_f(s1.x & 0xFFFFu);
  const uint32_t sh = s1.x >> 16, sl = s1.y;
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int ls = int(((sl >> (4 * j)) & 15) | (((sh >> (2 * j)) & 3) << 4)) - 32;
    acc = fmaf(float(iq4_group_dot<NG>(mw[j], xs, g0 + j)), (d * float(ls)) * xs.s2[g0 + j], acc);
  }
  return acc;
}

// Quantise one token's activation slice (U units, elements in natural order;
// pieces past the nu units in the slice are zero) into `xs`: the INT4
// kernels' fixed-point staging arithmetic (qnn_int4_dev.h), the 8 lanes of a
// 32-group meeting through DPP.  XIT float4 per thread.
template <int ENC, int U, int XIT>
__device__ __forceinline__ void stage_slice(XSlice<U * 8> &xs, const float4 (&xr)[XIT], int nu, int tid, int lane) {
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int e = (it * 256 + tid) * 4;
    const float4 v = e < nu * 256 ? xr[it] : make_float4(0.f, 0.f, 0.f, 0.f);
    const dev::GroupScale gs =
        dev::group_scale(dev::max_lanes8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)))));
    uint32_t b1[4], b2[4];
    dev::quant_elem(v.x, gs, b1[0], b2[0]);
    dev::quant_elem(v.y, gs, b1[1], b2[1]);
    dev::quant_elem(v.z, gs, b1[2], b2[2]);
    dev::quant_elem(v.w, gs, b1[3], b2[3]);
    uint32_t hw = dev::join2(dev::pack2(b1[0], b1[1]), dev::pack2(b1[2], b1[3]));
    uint32_t lw = dev::join2(dev::pack2(b2[0], b2[1]), dev::pack2(b2[2], b2[3]));
    if constexpr (ENC == QNN_WE_Q2_0) {  // 4x4 byte transpose over the quad of lanes holding a 16-element run
      hw = quad_transpose(hw, lane & 3);
      lw = quad_transpose(lw, lane & 3);
    }
    const int s16 = dev::sum_lanes4(dev::quant_sum<4>(b1, b2));  // 16-element sum
    const int s32 = s16 + int(dev::dpp<0x141>(uint32_t(s16)));
    if (e < U * 256) {
      const int g = e >> 5, k = (e >> 2) & 7;
      xs.h[g][k] = hw;
      xs.l[g][k] = lw;
      if ((lane & 3) == 0) xs.sum16[g][(lane >> 2) & 1] = s16;
      if ((lane & 7) == 0) {
        xs.s2[g] = gs.s1 * 0.00390625f;
        xs.sum32[g] = s32;
      }
    }
  }
}

// One unit's dot for format ENC (mw: main chunks; s1v, s1w, s2w: side fields;
// iq: the LDS codebook and sign masks of the IQ2/IQ3 formats).
template <int ENC, int NG>
__device__ __forceinline__ float unit_dot(const uint4 *mw, uint4 s1v, uint32_t s1w, uint32_t s2w,
                                          const XSlice<NG> &xs, int g0, const uint4 *iq) {
  if constexpr (ENC == QNN_WE_Q8_0) return unit_q8_0<NG>(mw, s1v, xs, g0);
  if constexpr (ENC == QNN_WE_Q4_K) return unit_q4_k<NG>(mw, xs, g0);
  if constexpr (ENC == QNN_WE_Q6_K) return unit_q6_k<NG>(mw, s1w, xs, g0);
  if constexpr (ENC == QNN_WE_Q3_K) return unit_q3_k<NG>(mw, s1v, s2w, xs, g0);
  if constexpr (ENC == QNN_WE_Q2_K) return unit_q2_k<NG>(mw, s1w, xs, g0);
  if constexpr (ENC == QNN_WE_Q5_K) return unit_q5_k<NG>(mw, xs, g0);
  if constexpr (ENC == QNN_WE_IQ4_NL) return unit_iq4_nl<NG>(mw, s1v, xs, g0);
  if constexpr (ENC == QNN_WE_IQ4_XS) return unit_iq4_xs<NG>(mw, s1v, xs, g0);
  if constexpr (ENC == QNN_WE_Q2_0) return unit_q2_0<NG>(mw, s1v, xs, g0);
  if constexpr (kIsIQ<ENC>) {
    constexpr int kGridU4 = kIQGridBytes<ENC> / 16;
    const uint64_t *mask = reinterpret_cast<const uint64_t *>(iq + kGridU4);
    const uint64_t *g64 = reinterpret_cast<const uint64_t *>(iq);
    const uint32_t *g32 = reinterpret_cast<const uint32_t *>(iq);
    if constexpr (ENC == QNN_WE_IQ2_XXS) return unit_iq2_xxs<NG>(mw, s1w, xs, g0, g64, mask);
    if constexpr (ENC == QNN_WE_IQ2_S) return unit_iq2_s<NG>(mw, s1w, xs, g0, g64, mask);
    if constexpr (ENC == QNN_WE_IQ3_XXS) return unit_iq3_xxs<NG>(mw, s1w, xs, g0, g32, mask);
    if constexpr (ENC == QNN_WE_IQ3_S) return unit_iq3_s<NG>(mw, s1v, s2w, xs, g0, g32, mask);
  }
  return 0.0f;
}

// Workgroup = 4 waves on one 64-row tile (SWIGLU: 32 gate rows in lanes
// 0-31, the same 32 up rows in lanes 32-63); slice = 4*BW units, wave w
// streams units [w*BW, (w+1)*BW) of it.
// A launch carries up to kGGMaxGroup such matvecs (the same input in
// practice: the q/k/v or gate/up projections of a layer); the member is
// chosen by workgroup range and computed exactly as on its own.
__device__ __forceinline__ int group_member(const GGGroup &grp) {
  int mi = 0;
  while (mi + 1 < grp.count && int(blockIdx.x) >= grp.start[mi + 1]) ++mi;
  return mi;
}
template <int ENC, int BW>
__device__ __forceinline__ void gguf_item(const GGGroup &grp, const int mi) {
  using F = Fmt<ENC>;
  constexpr int U = 4 * BW;   // units per slice
  constexpr int NG = U * 8;   // 32-groups per slice
  const GGArgs &a = grp.m[mi];
  const int slices = grp.slices[mi];
  const int bidx = int(blockIdx.x) - grp.start[mi];  // a multiple-of-8 offset keeps the XCD
  int tile, slice;
  if (!map_tile_slice(bidx, slices, a.tiles, tile, slice)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const GGLayout &l = a.l;
  const int u0 = slice * U;
  const int nu = min(U, l.units - u0);
  const int uw0 = wave * BW;
  const int nuw = max(0, min(BW, nu - uw0));

  // 1) activation slice (elements [u0*256, (u0+nu)*256) of token 0).  Loads
  //    are issued without per-lane branches (buffer loads past the row return
  //    0; pieces past the slice are zeroed when quantised), so the compiler
  //    can wait for them alone while the weight loads below are in flight.
  constexpr int XIT = (U * 256 + 1023) / 1024;
  float4 xr[XIT];
  const dev::Rsrc xsrc = dev::rsrc(a.x, size_t(l.cols) * 4);
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const uint32_t kb = uint32_t(u0 * 256 + (it * 256 + tid) * 4) * 4u;
    if (a.x_vec4) {  // uniform
      const uint4 v = dev::ld128(xsrc, kb, 0);
      xr[it] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    } else {
      xr[it] = make_float4(dev::ld32f(xsrc, kb, 0), dev::ld32f(xsrc, kb + 4, 0), dev::ld32f(xsrc, kb + 8, 0),
                           dev::ld32f(xsrc, kb + 12, 0));
    }
  }
  // 1b) IQ2/IQ3: the codebook and the sign masks, for LDS
  constexpr int kGridU4 = kIQGridBytes<ENC> / 16;
  constexpr int kTabU4 = kIsIQ<ENC> ? kGridU4 + kIQMaskU4<ENC> : 0;
  constexpr int kTabIt = (kTabU4 + 255) / 256;
  uint4 tr[kTabIt > 0 ? kTabIt : 1];
  if constexpr (kIsIQ<ENC>) {
    const uint4 *masks = iq_mask_src<ENC>();
#pragma unroll
    for (int it = 0; it < kTabIt; ++it) {  // every lane loads (pieces past the table re-read the last mask)
      const int t = it * 256 + tid;
      tr[it] = t < kGridU4 ? iq_grid_src<ENC>()[t] : masks[min(t - kGridU4, kIQMaskU4<ENC> - 1)];
    }
  }
  // 2) weights of this wave's units
  int stile = tile, srow = lane;
  const void *wb = a.w;
  if (a.mode >= GG_SWIGLU) {
    stile = tile >> 1;
    srow = (tile & 1) * 32 + (lane & 31);
    if (lane >= 32) wb = a.w2;
  }
  const Planes P = planes_of(l, wb);
  uint4 mw[BW][F::C];
  uint4 s1v[BW];
  uint32_t s1w[BW], s2w[BW];
  // Units past this wave's share re-read the slice's last unit (no per-unit
  // branch, so no load waits for another) and are skipped by the dot.
#pragma unroll
  for (int b = 0; b < BW; ++b) {
    const size_t tu = size_t(stile) * l.units + (u0 + min(uw0 + b, nu - 1));
    const uint4 *mp = reinterpret_cast<const uint4 *>(P.main) + (tu * F::C) * 64 + srow;
#pragma unroll
    for (int c = 0; c < F::C; ++c) mw[b][c] = wload(mp + c * 64);
    if (F::S1 == 16) s1v[b] = wload(reinterpret_cast<const uint4 *>(P.side1) + tu * 64 + srow);
    if (F::S1 == 8) {
      const uint2 *q = reinterpret_cast<const uint2 *>(P.side1) + tu * 64 + srow;
      const uint2 v = make_uint2(wload(reinterpret_cast<const uint32_t *>(q)), wload(reinterpret_cast<const uint32_t *>(q) + 1));
      s1v[b] = make_uint4(v.x, v.y, 0u, 0u);
    }
    if (F::S1 == 12) {
      const uint32_t *q = reinterpret_cast<const uint32_t *>(P.side1 + (tu * 64 + srow) * 12);
      s1v[b] = make_uint4(wload(q), wload(q + 1), wload(q + 2), 0u);
    }
    if (F::S1 == 4) s1w[b] = wload(reinterpret_cast<const uint32_t *>(P.side1) + tu * 64 + srow);
    if (F::S1 == 2) s1w[b] = wload(reinterpret_cast<const uint16_t *>(P.side1) + tu * 64 + srow);
    if (F::S2 == 2) s2w[b] = wload(reinterpret_cast<const uint16_t *>(P.side2) + tu * 64 + srow);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the quantisation below waits for x
  // 3) quantise the activation slice (natural element order)
  __shared__ XSlice<NG> xs;
  __shared__ float red[3][64];
  __shared__ uint4 iq_tab[kTabU4 > 0 ? kTabU4 : 1];
  if constexpr (kIsIQ<ENC>) {
#pragma unroll
    for (int it = 0; it < kTabIt; ++it)
      if (it * 256 + tid < kTabU4) iq_tab[it * 256 + tid] = tr[it];
  }
  stage_slice<ENC, U>(xs, xr, nu, tid, lane);
  __syncthreads();

  // 4) unit dots
  float acc = 0.0f;
#pragma unroll
  for (int b = 0; b < BW; ++b) {
    if (b < nuw) {
      const int g0 = (uw0 + b) * 8;
      if (ENC == QNN_WE_Q8_0) acc += unit_q8_0<NG>(mw[b], s1v[b], xs, g0);
      if (ENC == QNN_WE_Q4_K) acc += unit_q4_k<NG>(mw[b], xs, g0);
      if (ENC == QNN_WE_Q6_K) acc += unit_q6_k<NG>(mw[b], s1w[b], xs, g0);
      if (ENC == QNN_WE_Q3_K) acc += unit_q3_k<NG>(mw[b], s1v[b], s2w[b], xs, g0);
      if (ENC == QNN_WE_Q2_K) acc += unit_q2_k<NG>(mw[b], s1w[b], xs, g0);
      if (ENC == QNN_WE_Q5_K) acc += unit_q5_k<NG>(mw[b], xs, g0);
      if (ENC == QNN_WE_IQ4_NL) acc += unit_iq4_nl<NG>(mw[b], s1v[b], xs, g0);
      if (ENC == QNN_WE_IQ4_XS) acc += unit_iq4_xs<NG>(mw[b], s1v[b], xs, g0);
      if (ENC == QNN_WE_Q2_0) acc += unit_q2_0<NG>(mw[b], s1v[b], xs, g0);
      if constexpr (kIsIQ<ENC>) {
        const uint64_t *mask = reinterpret_cast<const uint64_t *>(iq_tab + kGridU4);
        const uint64_t *g64 = reinterpret_cast<const uint64_t *>(iq_tab);
        const uint32_t *g32 = reinterpret_cast<const uint32_t *>(iq_tab);
        if (ENC == QNN_WE_IQ2_XXS) acc += unit_iq2_xxs<NG>(mw[b], s1w[b], xs, g0, g64, mask);
        if (ENC == QNN_WE_IQ2_S) acc += unit_iq2_s<NG>(mw[b], s1w[b], xs, g0, g64, mask);
        if (ENC == QNN_WE_IQ3_XXS) acc += unit_iq3_xxs<NG>(mw[b], s1w[b], xs, g0, g32, mask);
        if (ENC == QNN_WE_IQ3_S) acc += unit_iq3_s<NG>(mw[b], s1v[b], s2w[b], xs, g0, g32, mask);
      }
    }
  }

  // 5) combine the 4 waves (fixed order), then split-K across workgroups
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave > 0) return;
  acc = ((acc + red[0][lane]) + red[1][lane]) + red[2][lane];
  if (slices > 1) {
    dev::xstore(a.partial + (size_t(tile) * slices + slice) * 64 + lane, acc);
    unsigned *ctr = &a.counters[size_t(tile) * kCounterStride];
    if (!dev::last_arrival(ctr, unsigned(slices), lane)) return;
    const float *pt = a.partial + size_t(tile) * slices * 64 + lane;
    float s[1];
    dev::sum_slices<1, 16>(s, [&](int sl, int) { return pt + size_t(sl) * 64; }, slices);
    acc = s[0];
    dev::reset_counter(ctr, lane);
  }
  // 6) epilogue
  if (a.mode >= GG_SWIGLU) {
    const float u = dev::xor_lanes<32>(acc);  // lanes 0-31 take 32-63
    const int row = tile * 32 + lane;
    if (lane < 32 && row < a.n) {
      if (a.g_out) {
        a.g_out[row] = acc;
        a.u_out[row] = u;
      }
      a.y[row] = (a.mode == GG_GEGLU ? gelu_dev(acc) : silu_dev(acc)) * u;
    }
  } else {
    const int row = tile * 64 + lane;
    if (row < a.n) a.y[row] = acc;
  }
}

template <int ENC, int BW>
__global__ __launch_bounds__(256) void k_gguf_matvec(const GGGroup grp) {
  gguf_item<ENC, BW>(grp, group_member(grp));
}
// The IQ2/IQ3 matvecs at one unit per wave, held to 128 VGPRs (4 waves per
// SIMD): IQ2_S at 14336 x 3584 (3.5 workgroups per CU) measured 14.8 us at
// the compiler's own 130 VGPRs (3 waves per SIMD) and 13.8 us so.
template <int ENC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_gguf_matvec_iq(const GGGroup grp) {
  gguf_item<ENC, 1>(grp, group_member(grp));
}
// Up to MT tokens (rows of x, `ntok` valid, the rest zero) in one pass over
// the weights: a Linear of a few rows, MT at a time.  The
// workgroup and plan are the one-token kernel's at one unit per wave; each
// token has its own activation slice in LDS, the wave's unit is loaded once
// and dotted with every slice, and the split-K exchange carries MT partial
// sums per row.  Per token the arithmetic is the one-token kernel's.
template <int ENC, int MT>
__global__ __launch_bounds__(256) void k_gguf_matvec_mt(const GGArgs a, int slices, int ntok) {
  using F = Fmt<ENC>;
  constexpr int U = 4, NG = U * 8;
  int tile, slice;
  if (!map_tile_slice(int(blockIdx.x), slices, a.tiles, tile, slice)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const GGLayout &l = a.l;
  const int u0 = slice * U, nu = min(U, l.units - u0);
  const bool on = wave < nu;

  // 1) the tokens' activation slices (buffer loads past the last token read 0)
  float4 xr[MT][1];
  const dev::Rsrc xsrc = dev::rsrc(a.x, size_t(ntok) * l.cols * 4);
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint32_t kb = uint32_t(size_t(m) * l.cols * 4 + size_t(u0 * 256 + tid * 4) * 4);
    if (a.x_vec4) {
      const uint4 v = dev::ld128(xsrc, kb, 0);
      xr[m][0] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    } else {
      xr[m][0] = make_float4(dev::ld32f(xsrc, kb, 0), dev::ld32f(xsrc, kb + 4, 0), dev::ld32f(xsrc, kb + 8, 0),
                             dev::ld32f(xsrc, kb + 12, 0));
    }
  }
  // 1b) IQ2/IQ3: the codebook and the sign masks, for LDS
  constexpr int kGridU4 = kIQGridBytes<ENC> / 16;
  constexpr int kTabU4 = kIsIQ<ENC> ? kGridU4 + kIQMaskU4<ENC> : 0;
  constexpr int kTabIt = (kTabU4 + 255) / 256;
  uint4 tr[kTabIt > 0 ? kTabIt : 1];
  if constexpr (kIsIQ<ENC>) {
    const uint4 *masks = iq_mask_src<ENC>();
#pragma unroll
    for (int it = 0; it < kTabIt; ++it) {
      const int t = it * 256 + tid;
      tr[it] = t < kGridU4 ? iq_grid_src<ENC>()[t] : masks[min(t - kGridU4, kIQMaskU4<ENC> - 1)];
    }
  }
  // 2) this wave's unit (past the slice's units: its last unit, unused)
  const Planes P = planes_of(l, a.w);
  uint4 mw[F::C];
  uint4 s1v = make_uint4(0u, 0u, 0u, 0u);
  uint32_t s1w = 0, s2w = 0;
  {
    const size_t tu = size_t(tile) * l.units + (u0 + min(wave, nu - 1));
    const uint4 *mp = reinterpret_cast<const uint4 *>(P.main) + (tu * F::C) * 64 + lane;
#pragma unroll
    for (int c = 0; c < F::C; ++c) mw[c] = wload(mp + c * 64);
    if (F::S1 == 16) s1v = wload(reinterpret_cast<const uint4 *>(P.side1) + tu * 64 + lane);
    if (F::S1 == 8) {
      const uint32_t *q = reinterpret_cast<const uint32_t *>(P.side1) + (tu * 64 + lane) * 2;
      s1v = make_uint4(wload(q), wload(q + 1), 0u, 0u);
    }
    if (F::S1 == 12) {
      const uint32_t *q = reinterpret_cast<const uint32_t *>(P.side1 + (tu * 64 + lane) * 12);
      s1v = make_uint4(wload(q), wload(q + 1), wload(q + 2), 0u);
    }
    if (F::S1 == 4) s1w = wload(reinterpret_cast<const uint32_t *>(P.side1) + tu * 64 + lane);
    if (F::S1 == 2) s1w = wload(reinterpret_cast<const uint16_t *>(P.side1) + tu * 64 + lane);
    if (F::S2 == 2) s2w = wload(reinterpret_cast<const uint16_t *>(P.side2) + tu * 64 + lane);
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3) the slices into LDS
  __shared__ XSlice<NG> xs[MT];
  __shared__ float red[4][MT][64];
  __shared__ uint4 iq_tab[kTabU4 > 0 ? kTabU4 : 1];
  if constexpr (kIsIQ<ENC>) {
#pragma unroll
    for (int it = 0; it < kTabIt; ++it)
      if (it * 256 + tid < kTabU4) iq_tab[it * 256 + tid] = tr[it];
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) stage_slice<ENC, U>(xs[m], xr[m], nu, tid, lane);
  __syncthreads();
  // 4) the unit against every valid token, one token at a time (the loop is
  //    kept rolled: unrolled, the compiler holds every token's unpacked
  //    weights at once, 256 VGPRs and one wave per SIMD)
#pragma unroll 1
  for (int m = 0; m < ntok; ++m)
    red[wave][m][lane] = on ? unit_dot<ENC, NG>(mw, s1v, s1w, s2w, xs[m], wave * 8, iq_tab) : 0.0f;
  // 5) the 4 waves (fixed order), then split-K across workgroups
  __syncthreads();
  if (wave > 0) return;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
    acc[m] = m < ntok ? ((red[0][m][lane] + red[1][m][lane]) + red[2][m][lane]) + red[3][m][lane] : 0.0f;
  if (slices > 1) {
#pragma unroll
    for (int m = 0; m < MT; ++m) dev::xstore(a.partial + ((size_t(tile) * slices + slice) * MT + m) * 64 + lane, acc[m]);
    unsigned *ctr = &a.counters[size_t(tile) * kCounterStride];
    if (!dev::last_arrival(ctr, unsigned(slices), lane)) return;
    const float *pt = a.partial + size_t(tile) * slices * MT * 64 + lane;
    dev::sum_slices<MT, 4>(acc, [&](int sl, int m) { return pt + (size_t(sl) * MT + m) * 64; }, slices);
    dev::reset_counter(ctr, lane);
  }
  // 6) y rows of the valid tokens
  const int row = tile * 64 + lane;
  if (row < a.n)
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (m < ntok) a.y[size_t(m) * a.n + row] = acc[m];
}

// Members of two K-quant encodings in one launch (a layer's q/k/v often mix
// quant types), one unit per wave; each workgroup runs its member's own code.
template <int E0, int E1>
__global__ __launch_bounds__(256) void k_gguf_matvec_mixed(const GGGroup grp) {
  const int mi = group_member(grp);
  if (grp.m[mi].l.enc == E0) gguf_item<E0, 1>(grp, mi);
  else gguf_item<E1, 1>(grp, mi);
}

template <int E0>
void launch_mixed(const GGGroup &g, int e1, hipStream_t st) {
  const int grid = g.start[g.count];
  switch (e1) {
    case QNN_WE_Q4_K:
      if constexpr (E0 != QNN_WE_Q4_K) {
        hipLaunchKernelGGL((k_gguf_matvec_mixed<E0, QNN_WE_Q4_K>), dim3(grid), dim3(256), 0, st, g);
        return;
      }
      break;
    case QNN_WE_Q6_K:
      if constexpr (E0 != QNN_WE_Q6_K) {
        hipLaunchKernelGGL((k_gguf_matvec_mixed<E0, QNN_WE_Q6_K>), dim3(grid), dim3(256), 0, st, g);
        return;
      }
      break;
    case QNN_WE_Q3_K:
      if constexpr (E0 != QNN_WE_Q3_K) {
        hipLaunchKernelGGL((k_gguf_matvec_mixed<E0, QNN_WE_Q3_K>), dim3(grid), dim3(256), 0, st, g);
        return;
      }
      break;
    case QNN_WE_Q2_K:
      if constexpr (E0 != QNN_WE_Q2_K) {
        hipLaunchKernelGGL((k_gguf_matvec_mixed<E0, QNN_WE_Q2_K>), dim3(grid), dim3(256), 0, st, g);
        return;
      }
      break;
    default: break;
  }
  fail(QNN_E_INVALID_OP, "gguf mixed group encodings");
}

template <int ENC>
void launch_enc(const GGGroup &g, int bw, hipStream_t st) {
  const int grid = g.start[g.count];
  if (kIsIQ<ENC> && bw == 1) hipLaunchKernelGGL((k_gguf_matvec_iq<ENC>), dim3(grid), dim3(256), 0, st, g);
  else if (bw == 2) hipLaunchKernelGGL((k_gguf_matvec<ENC, 2>), dim3(grid), dim3(256), 0, st, g);
  else hipLaunchKernelGGL((k_gguf_matvec<ENC, 1>), dim3(grid), dim3(256), 0, st, g);
}

}  // namespace

GGLayout gguf_layout(int enc, int rows, int cols) {
  GGLayout l;
  l.enc = enc;
  l.rows = rows;
  l.cols = cols;
  l.tiles = (rows + 63) / 64;
  l.units = (cols + 255) / 256;
  switch (enc) {
    case QNN_WE_Q4_K: l.main_chunks = 9; l.side1_bytes = 0; l.side2_bytes = 0; l.unit_bytes = 144; break;
    case QNN_WE_Q6_K: l.main_chunks = 13; l.side1_bytes = 2; l.side2_bytes = 0; l.unit_bytes = 210; break;
    case QNN_WE_Q3_K: l.main_chunks = 6; l.side1_bytes = 12; l.side2_bytes = 2; l.unit_bytes = 110; break;
    case QNN_WE_Q2_K: l.main_chunks = 5; l.side1_bytes = 4; l.side2_bytes = 0; l.unit_bytes = 84; break;
    case QNN_WE_Q8_0: l.main_chunks = 16; l.side1_bytes = 16; l.side2_bytes = 0; l.unit_bytes = 272; break;
    case QNN_WE_Q5_K: l.main_chunks = 11; l.side1_bytes = 0; l.side2_bytes = 0; l.unit_bytes = 176; break;
    case QNN_WE_IQ4_XS: l.main_chunks = 8; l.side1_bytes = 8; l.side2_bytes = 0; l.unit_bytes = 136; break;
    case QNN_WE_IQ4_NL: l.main_chunks = 8; l.side1_bytes = 16; l.side2_bytes = 0; l.unit_bytes = 144; break;
    case QNN_WE_Q2_0: l.main_chunks = 4; l.side1_bytes = 8; l.side2_bytes = 0; l.unit_bytes = 72; break;
    case QNN_WE_IQ2_XXS: l.main_chunks = 4; l.side1_bytes = 2; l.side2_bytes = 0; l.unit_bytes = 66; break;
    case QNN_WE_IQ2_S: l.main_chunks = 5; l.side1_bytes = 2; l.side2_bytes = 0; l.unit_bytes = 82; break;
    case QNN_WE_IQ3_XXS: l.main_chunks = 6; l.side1_bytes = 2; l.side2_bytes = 0; l.unit_bytes = 98; break;
    case QNN_WE_IQ3_S: l.main_chunks = 6; l.side1_bytes = 12; l.side2_bytes = 2; l.unit_bytes = 110; break;
    default: fail(QNN_E_NOT_SUPPORTED, "GGUF encoding not supported by the HIP backend");
  }
  l.src_row_bytes = enc == QNN_WE_Q8_0     ? (cols / 32) * 34
                    : enc == QNN_WE_IQ4_NL ? (cols / 32) * 18
                    : enc == QNN_WE_Q2_0   ? (cols / 64) * 18
                                           : (cols / 256) * l.unit_bytes;
  const size_t tu64 = size_t(l.tiles) * l.units * 64;
  auto up256 = [](size_t b) { return (b + 255) & ~size_t(255); };
  l.side1_off = up256(tu64 * l.main_chunks * 16);
  l.side2_off = l.side1_off + up256(tu64 * l.side1_bytes);
  l.total = l.side2_off + up256(tu64 * l.side2_bytes);
  if (enc == QNN_WE_Q8_0) {
    l.rowexp_off = l.total;
    l.total += up256(size_t(l.tiles) * 64 * 4);
  }
  return l;
}

void gguf_repack_launch(const uint8_t *src, const GGLayout &l, void *dst, hipStream_t s) {
  const size_t total = size_t(l.tiles) * l.units * 64;
  hipLaunchKernelGGL(k_gguf_repack, dim3((total + 255) / 256), dim3(256), 0, s, src, l, static_cast<uint8_t *>(dst));
  hip_check(hipGetLastError(), "gguf repack launch");
}

void gguf_dequant_launch(const GGLayout &l, const void *w, float *out, hipStream_t s) {
  const size_t total = size_t(l.rows) * l.cols;
  hipLaunchKernelGGL(k_gguf_dequant, dim3((total + 255) / 256), dim3(256), 0, s, l,
                     static_cast<const uint8_t *>(w), out);
  hip_check(hipGetLastError(), "gguf dequant launch");
}

void gguf_gather_launch(const GGLayout &l, const void *w, const float *ids, float *out, int rows, int vocab,
                        hipStream_t s) {
  const size_t total = size_t(rows) * l.cols;
  hipLaunchKernelGGL(k_gguf_gather, dim3((total + 255) / 256), dim3(256), 0, s, l, static_cast<const uint8_t *>(w),
                     reinterpret_cast<const unsigned *>(ids), out, rows, vocab);
  hip_check(hipGetLastError(), "gguf gather launch");
}

void gguf_rowexp_launch(const GGLayout &l, const void *w, int *ew, int rows_pad, hipStream_t s) {
  hipLaunchKernelGGL(k_gguf_rowexp, dim3(rows_pad), dim3(256), 0, s, l, static_cast<const uint8_t *>(w), ew);
  hip_check(hipGetLastError(), "gguf row exponents");
}

void gguf_expand_h16_launch(const GGLayout &l, const void *w, const int *ew, void *out, hipStream_t s) {
  const int ksteps = (l.cols + 63) / 64 * 4;
  const size_t pieces = q8_h16_bytes(l.rows, l.cols) / 16;
  hipLaunchKernelGGL(k_gguf_expand_h16, dim3((pieces + 255) / 256), dim3(256), 0, s, l,
                     static_cast<const uint8_t *>(w), ew, ksteps, pieces, static_cast<uint4 *>(out));
  hip_check(hipGetLastError(), "gguf fp16 expansion");
}

void gguf_plan(const GGLayout &l, int tiles, int *bw, int *slices) {
  (void)tiles;
  const int forced = tuning().gg_bw;
  // One unit per wave at every shape: the Gemma-2 Q6_K head (256000 x 3584,
  // 64k waves) measured 134.4 us against 145.2 us at two units per wave, its
  // down projection 13.1 against 13.8 us.  QNN_GG_BW=2 selects two.
  int pick = 1;
  if (forced == 1 || forced == 2) pick = forced;
  *bw = pick;
  *slices = (l.units + 4 * pick - 1) / (4 * pick);
}

void gguf_group_launch(const GGGroup &g, int bw, hipStream_t s) {
  if (g.count < 1 || g.count > kGGMaxGroup) fail(QNN_E_INVALID_OP, "gguf group size");
  int e1 = g.m[0].l.enc;
  for (int i = 1; i < g.count; ++i)
    if (g.m[i].l.enc != g.m[0].l.enc) e1 = g.m[i].l.enc;
  if (e1 != g.m[0].l.enc) {  // two encodings (the recorder allows at most two K-quants, one unit per wave)
    if (bw != 1) fail(QNN_E_INVALID_OP, "gguf mixed group width");
    switch (g.m[0].l.enc) {
      case QNN_WE_Q4_K: launch_mixed<QNN_WE_Q4_K>(g, e1, s); break;
      case QNN_WE_Q6_K: launch_mixed<QNN_WE_Q6_K>(g, e1, s); break;
      case QNN_WE_Q3_K: launch_mixed<QNN_WE_Q3_K>(g, e1, s); break;
      case QNN_WE_Q2_K: launch_mixed<QNN_WE_Q2_K>(g, e1, s); break;
      default: fail(QNN_E_INVALID_OP, "gguf mixed group encodings");
    }
    hip_check(hipGetLastError(), "gguf matvec launch");
    return;
  }
  switch (g.m[0].l.enc) {
    case QNN_WE_Q4_K: launch_enc<QNN_WE_Q4_K>(g, bw, s); break;
    case QNN_WE_Q6_K: launch_enc<QNN_WE_Q6_K>(g, bw, s); break;
    case QNN_WE_Q3_K: launch_enc<QNN_WE_Q3_K>(g, bw, s); break;
    case QNN_WE_Q2_K: launch_enc<QNN_WE_Q2_K>(g, bw, s); break;
    case QNN_WE_Q8_0: launch_enc<QNN_WE_Q8_0>(g, bw, s); break;
    case QNN_WE_Q5_K: launch_enc<QNN_WE_Q5_K>(g, bw, s); break;
    case QNN_WE_IQ4_NL: launch_enc<QNN_WE_IQ4_NL>(g, bw, s); break;
    case QNN_WE_IQ4_XS: launch_enc<QNN_WE_IQ4_XS>(g, bw, s); break;
    case QNN_WE_Q2_0: launch_enc<QNN_WE_Q2_0>(g, bw, s); break;
    case QNN_WE_IQ2_XXS: launch_enc<QNN_WE_IQ2_XXS>(g, bw, s); break;
    case QNN_WE_IQ2_S: launch_enc<QNN_WE_IQ2_S>(g, bw, s); break;
    case QNN_WE_IQ3_XXS: launch_enc<QNN_WE_IQ3_XXS>(g, bw, s); break;
    case QNN_WE_IQ3_S: launch_enc<QNN_WE_IQ3_S>(g, bw, s); break;
    default: fail(QNN_E_NOT_SUPPORTED, "GGUF encoding not supported by the HIP backend");
  }
  hip_check(hipGetLastError(), "gguf matvec launch");
}

void gguf_matvec_mt_launch(const GGArgs &a, int slices, int ntok, hipStream_t s) {
  if (ntok < 1 || ntok > kGGMaxTokens) fail(QNN_E_INVALID_OP, "gguf multi-token width");
  const int grid = (a.tiles + 7) / 8 * 8 * slices;
#define QNN_GG_MT(E) hipLaunchKernelGGL((k_gguf_matvec_mt<E, kGGMaxTokens>), dim3(grid), dim3(256), 0, s, a, slices, ntok)
  switch (a.l.enc) {
    case QNN_WE_Q4_K: QNN_GG_MT(QNN_WE_Q4_K); break;
    case QNN_WE_Q6_K: QNN_GG_MT(QNN_WE_Q6_K); break;
    case QNN_WE_Q3_K: QNN_GG_MT(QNN_WE_Q3_K); break;
    case QNN_WE_Q2_K: QNN_GG_MT(QNN_WE_Q2_K); break;
    case QNN_WE_Q8_0: QNN_GG_MT(QNN_WE_Q8_0); break;
    case QNN_WE_Q5_K: QNN_GG_MT(QNN_WE_Q5_K); break;
    case QNN_WE_IQ4_NL: QNN_GG_MT(QNN_WE_IQ4_NL); break;
    case QNN_WE_IQ4_XS: QNN_GG_MT(QNN_WE_IQ4_XS); break;
    case QNN_WE_Q2_0: QNN_GG_MT(QNN_WE_Q2_0); break;
    case QNN_WE_IQ2_XXS: QNN_GG_MT(QNN_WE_IQ2_XXS); break;
    case QNN_WE_IQ2_S: QNN_GG_MT(QNN_WE_IQ2_S); break;
    case QNN_WE_IQ3_XXS: QNN_GG_MT(QNN_WE_IQ3_XXS); break;
    case QNN_WE_IQ3_S: QNN_GG_MT(QNN_WE_IQ3_S); break;
    default: fail(QNN_E_NOT_SUPPORTED, "GGUF encoding not supported by the HIP backend");
  }
#undef QNN_GG_MT
  hip_check(hipGetLastError(), "gguf multi-token matvec launch");
}

void gguf_matvec_launch(const GGArgs &a, int bw, int slices, hipStream_t s) {
  GGGroup g;
  g.m[0] = a;
  g.slices[0] = slices;
  g.start[0] = 0;
  g.start[1] = (a.tiles + 7) / 8 * 8 * slices;
  g.count = 1;
  gguf_group_launch(g, bw, s);
}

}  // namespace qnn
