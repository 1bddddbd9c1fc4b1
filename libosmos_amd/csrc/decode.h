// libosmos MI355X - the GGUF blocks' exact fp32 values, 8 at a time (chunk k: values 8k .. 8k + 7 of a block). The
// values are the reference's (kernels/quant.h:60-348, gguf-py's dequantize); shared by mv.hip (the fp32 matvec),
// mm.hip (the f16 matmul) and quant.hip (quant_dequant).
//
// Design: every quantized format here is "a small integer code per value, times a float scale, minus a float minimum"
// (the IQ1 types: "times a scale, of the code plus a float delta"). So a type's decoder does integer work only: it
// reads the chunk's header fields and produces a Chunk - the 8 codes packed as bit fields at byte stride in two 32-bit
// words, built 4 at a time with packed shifts, masks and xors - and the chunk's float scale and minimum. One shared
// epilogue (`finish`) turns a Chunk into the 8 floats with the type's float steps, each rounded on its own
// (__fmul_rn / __fsub_rn / __fadd_rn, never contracted), so the bits are the reference's:
//   plain:  v = scale * (float) code                       (Q8_0, Q4_0, Q6_K, Q3_K, IQ4_NL, IQ4_XS, IQ2_*, IQ3_XXS)
//   min:    v = (scale * (float) code) - minimum           (Q2_K, Q4_K, Q5_K)
//   delta:  v = scale * ((float) code + delta)             (IQ1_S, IQ1_M)
// Signed codes whose format stores an offset form (q - 8, q - 32, q - 4) are kept as a field of width b holding
// (q xor 2^(b-1)): sign-extending that field is exactly q - 2^(b-1), so the epilogue's one bit-field extract
// (v_bfe_i32) gives the signed code with no per-value subtract. The IQ grids' signs are applied to all 4 bytes of a
// word at once: (g xor m) + (m & 1) with m = 0xFF in the negated bytes (grid bytes are never 0, so no carry crosses
// a byte). A negated code gives the negated product (round-to-nearest is symmetric), the reference's -x.
#pragma once
#include "common.h"

namespace osm {

constexpr int kChunk = 8;

struct DecodeTables {
  Grids g;
  int8_t iq4nl[16];
};

constexpr DecodeTables make_decode_tables() {
  DecodeTables t{};
  t.g = make_grids();
  constexpr int8_t v[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
  for (int i = 0; i < 16; i++) t.iq4nl[i] = v[i];
  return t;
}

// the float form of a type's codes (the epilogue's steps)
enum class Form { kPlain, kMin, kDelta };

// one decoded chunk: code j is the `Bits`-wide field at bit 8 (j % 4) of word j / 4, signed or not per the type
struct Chunk {
  uint32_t w[2];
  float scale, second;  // `second`: the minimum (kMin) or the delta (kDelta)
};

// per type: the code fields' width and signedness and the float form
template <uint32_t T> struct Codec;
#define OSM_CODEC(t, bits, sgn, form) \
  template <> struct Codec<t> { static constexpr int kBits = bits; static constexpr bool kSigned = sgn; \
                                static constexpr Form kForm = form; };
OSM_CODEC(kQ8_0, 8, true, Form::kPlain)
OSM_CODEC(kQ4_0, 4, true, Form::kPlain)     // q - 8 as (q ^ 8), 4 bits
OSM_CODEC(kIQ4_NL, 8, true, Form::kPlain)
OSM_CODEC(kIQ4_XS, 8, true, Form::kPlain)
OSM_CODEC(kQ6_K, 6, true, Form::kPlain)     // q - 32 as (q ^ 32), 6 bits
OSM_CODEC(kQ3_K, 3, true, Form::kPlain)     // q2 + 4 hbit - 4 as ((q2 | hbit << 2) ^ 4), 3 bits
OSM_CODEC(kQ2_K, 2, false, Form::kMin)
OSM_CODEC(kQ4_K, 4, false, Form::kMin)
OSM_CODEC(kQ5_K, 5, false, Form::kMin)
OSM_CODEC(kQ5_KR, 5, false, Form::kMin)
OSM_CODEC(kIQ2_XXS, 8, true, Form::kPlain)
OSM_CODEC(kIQ2_XS, 8, true, Form::kPlain)
OSM_CODEC(kIQ2_S, 8, true, Form::kPlain)
OSM_CODEC(kIQ3_XXS, 8, true, Form::kPlain)
OSM_CODEC(kIQ1_S, 8, true, Form::kDelta)
OSM_CODEC(kIQ1_M, 8, true, Form::kDelta)
#undef OSM_CODEC

__device__ inline float mul(float a, float b) { return __fmul_rn(a, b); }

template <uint32_t T>
__device__ inline void finish(const Chunk& c, float* v) {
  constexpr int B = Codec<T>::kBits;
#pragma unroll
  for (int j = 0; j < kChunk; j++) {
    const uint32_t word = c.w[j / 4];
    const int q = Codec<T>::kSigned ? __builtin_amdgcn_sbfe((int) word, 8 * (j % 4), B)
                                    : (int) __builtin_amdgcn_ubfe(word, 8 * (j % 4), B);
    if constexpr (Codec<T>::kForm == Form::kPlain) v[j] = mul(c.scale, (float) q);
    else if constexpr (Codec<T>::kForm == Form::kMin) v[j] = __fsub_rn(mul(c.scale, (float) q), c.second);
    else v[j] = mul(c.scale, __fadd_rn((float) q, c.second));
  }
}

// ---- packed helpers: 4 codes a word ----
constexpr uint32_t kEach = 0x01010101u;  // one in every byte

// a 4-bit sign nibble as a byte mask (0xFF where the bit is set): each bit moved to its byte's bit 0, then x 0xFF
__device__ inline uint32_t sign_bytes(uint32_t nib) { return ((nib & 0xFu) * 0x00204081u & kEach) * 0xFFu; }
// 4 unsigned grid bytes, negated where `nib` says: two's complement a byte, no carries (every grid byte is >= 1)
__device__ inline uint32_t apply_signs(uint32_t g, uint32_t nib) {
  const uint32_t m = sign_bytes(nib);
  return (g ^ m) + (m & kEach);
}
__device__ inline void signed_grid(Chunk& c, uint64_t grid, uint32_t signs8) {
  c.w[0] = apply_signs((uint32_t) grid, signs8);
  c.w[1] = apply_signs((uint32_t) (grid >> 32), signs8 >> 4);
}
// the IQ4 non-linear table as 4 little-endian words (entry i at byte i % 4 of word i / 4)
constexpr uint32_t iq4_word(int w) {
  uint32_t r = 0;
  for (int b = 0; b < 4; b++) r |= (uint32_t) (uint8_t) make_decode_tables().iq4nl[4 * w + b] << (8 * b);
  return r;
}
// 4 bytes from the IQ4 table, indexed by 4 nibbles at `shift` of the bytes of `idx`: entries 0-7 and 8-15 each one
// byte permute of two table words, then the index's bit 3 picks between them per byte (no memory lookups)
template <typename Tab>
__device__ inline uint32_t table4(const Tab&, uint32_t idx, int shift) {
  const uint32_t n = (idx >> shift) & 0x0F0F0F0Fu, sel = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(iq4_word(1), iq4_word(0), sel);
  const uint32_t hi = __builtin_amdgcn_perm(iq4_word(3), iq4_word(2), sel);
  const uint32_t m = ((n >> 3) & 0x01010101u) * 0xFFu;
  return (hi & m) | (lo & ~m);
}
__device__ inline uint32_t nibbles(uint32_t word, int shift) { return (word >> shift) & (0x0Fu * kEach); }
__device__ inline float half_at(const uint8_t* p) { return f16(ld16(p)); }

// the 6-bit scale and minimum of 32-value group g (of 8) in the K-quants' 12-byte table: bytes 0-3 hold the low six
// bits of scales 0-3, bytes 4-7 those of minimums 0-3; groups 4-7 take their low nibbles from bytes 8-11 (scale: low,
// minimum: high) and their top two bits from the top bits of bytes g - 4 (scale) and g (minimum)
__device__ inline void group_scale_min(const uint8_t* t, int g, uint32_t& sc, uint32_t& mn) {
  if (g < 4) {
    sc = t[g] & 63u, mn = t[g + 4] & 63u;
  } else {
    const uint32_t packed = t[g + 4], top_s = t[g - 4] >> 6, top_m = t[g] >> 6;
    sc = (packed & 15u) | top_s << 4, mn = (packed >> 4) | top_m << 4;
  }
}

// ---- per type: Layout<T>::at(tables, block, chunk k) -> Chunk ----
template <uint32_t T> struct Layout;

// Q8_0: f16 d, 32 int8 (chunk k: bytes 2 + 8k ..)
template <> struct Layout<kQ8_0> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    return Chunk{{ld32(b + 2 + 8 * k), ld32(b + 6 + 8 * k)}, half_at(b), 0.0f};
  }
};
// Q4_0: f16 d, 16 bytes of nibbles: values 0-15 the low nibbles, 16-31 the high
template <> struct Layout<kQ4_0> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const uint8_t* q = b + 2 + 8 * (k & 1);
    const int sh = 4 * (k >> 1);
    return Chunk{{nibbles(ld32(q), sh) ^ 8u * kEach, nibbles(ld32(q + 4), sh) ^ 8u * kEach}, half_at(b), 0.0f};
  }
};
// IQ4_NL: f16 d, nibble indices (Q4_0's order) into the 16-entry non-linear table
template <> struct Layout<kIQ4_NL> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const uint8_t* q = b + 2 + 8 * (k & 1);
    const int sh = 4 * (k >> 1);
    return Chunk{{table4(K, ld32(q), sh), table4(K, ld32(q + 4), sh)}, half_at(b), 0.0f};
  }
};
// IQ4_XS: f16 d, u16 scale high bits, 4 bytes of scale low nibbles, 128 bytes of nibble indices (16 a 32-group:
// values 0-15 the low nibbles, 16-31 the high); group scale (6 bits) - 32
template <> struct Layout<kIQ4_XS> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const int g = k >> 2, half = (k >> 1) & 1;
    const uint32_t lo4 = (b[4 + (g >> 1)] >> (4 * (g & 1))) & 15u, hi2 = (ld16(b + 2) >> (2 * g)) & 3u;
    const uint8_t* q = b + 8 + 16 * g + 8 * (k & 1);
    return Chunk{{table4(K, ld32(q), 4 * half), table4(K, ld32(q + 4), 4 * half)},
                 mul(half_at(b), (float) ((int) (lo4 | hi2 << 4) - 32)), 0.0f};
  }
};
// Q4_K: f16 d, f16 dmin, 12 scale bytes, 128 nibble bytes (32-groups 2i and 2i + 1 share bytes 32i .. 32i + 31: low
// and high nibbles)
template <> struct Layout<kQ4_K> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const int g = k >> 2;
    uint32_t sc, mn;
    group_scale_min(b + 4, g, sc, mn);
    const uint8_t* q = b + 16 + 32 * (g >> 1) + 8 * (k & 3);
    const int sh = 4 * (g & 1);
    return Chunk{{nibbles(ld32(q), sh), nibbles(ld32(q + 4), sh)}, mul(half_at(b), (float) sc),
                 mul(half_at(b + 2), (float) mn)};
  }
};
// Q5_K: Q4_K's header, 32 bytes of fifth bits (bit g of byte l: value l of group g), then Q4_K's nibbles
template <> struct Layout<kQ5_K> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const int g = k >> 2;
    uint32_t sc, mn;
    group_scale_min(b + 4, g, sc, mn);
    const uint8_t *h = b + 16 + 8 * (k & 3), *q = b + 48 + 32 * (g >> 1) + 8 * (k & 3);
    const int sh = 4 * (g & 1);
    Chunk c{{0, 0}, mul(half_at(b), (float) sc), mul(half_at(b + 2), (float) mn)};
#pragma unroll
    for (int i = 0; i < 2; i++) c.w[i] = nibbles(ld32(q + 4 * i), sh) | ((ld32(h + 4 * i) >> g) & kEach) << 4;
    return c;
  }
};
// Q5_KR, Q5_K repacked (the reference's layout, include/osmos/gpu/quant.h:17-19,42-47, kernels/quant.h:117-123): rows
// in tiles of 16; a tile's block of 256 columns is 2880 bytes - the 16 rows' f16 d and dmin (4 bytes a row), then for
// each 32-value group g a 352-byte segment: 32 slots of 16 values (slot h 16 + r: row r's chunks 4 g + h and
// 4 g + 2 + h) as 8 bytes of low nibbles (value i at nibble i) at slot 8, their fifth bits as 2 bytes at
// 256 + slot 2, then each row's 6-bit scale and minimum as 2 bytes at 320 + r 2. `b` is the tile's block and chunk k
// is r 32 + c (row r's chunk c): the same fields as Q5_K's, so the same values
template <> struct Layout<kQ5_KR> {
  static constexpr int kRows = 16, kHead = 64, kSeg = 352, kHighs = 256, kScales = 320;
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const int r = k >> 5, c = k & 31, g = c >> 2, h = c & 1, upper = (c >> 1) & 1, slot = h * kRows + r;
    const uint8_t* seg = b + kHead + g * kSeg;
    const uint32_t nib = ld32(seg + slot * 8 + 4 * upper);             // this chunk's 8 nibbles
    const uint32_t hi = (ld16(seg + kHighs + slot * 2) >> (8 * upper)) & 0xFFu;  // and their fifth bits
    const uint32_t sm = ld16(seg + kScales + r * 2);
    // nibble i to byte i % 4 of word i / 4: spread each 16-bit half's 4 nibbles over 4 bytes
    auto spread = [](uint32_t x) { x = (x | x << 8) & 0x00FF00FFu; return (x | x << 4) & 0x0F0F0F0Fu; };
    // fifth bit i to bit 4 of byte i % 4 of word i / 4
    auto highs = [](uint32_t x) { return ((x & 0xFu) * 0x00204081u & kEach) << 4; };
    return Chunk{{spread(nib & 0xFFFFu) | highs(hi), spread(nib >> 16) | highs(hi >> 4)},
                 mul(half_at(b + 4 * r), (float) (sm & 0xFFu)), mul(half_at(b + 4 * r + 2), (float) (sm >> 8))};
  }
};
// Q6_K: 128 bytes of low nibbles, 64 bytes of 2-bit highs, 16 int8 scales (one a 16 values), f16 d. Values are in
// halves of 128: value 128 h + 32 r + l (r < 4, l < 32) has its low nibble in byte 64 h + 32 (r & 1) + l (high nibble
// for r >= 2) and its high pair at bits 2r of byte 128 + 32 h + l
template <> struct Layout<kQ6_K> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const int v0 = 8 * k, h = v0 >> 7, r = (v0 >> 5) & 3, l = v0 & 31;
    const uint8_t *lo = b + 64 * h + 32 * (r & 1) + l, *hi = b + 128 + 32 * h + l;
    Chunk c{{0, 0}, mul(half_at(b + 208), (float) (int8_t) b[192 + (v0 >> 4)]), 0.0f};
#pragma unroll
    for (int i = 0; i < 2; i++)
      c.w[i] = (nibbles(ld32(lo + 4 * i), 4 * (r >> 1)) | ((ld32(hi + 4 * i) >> (2 * r)) & 3u * kEach) << 4) ^ 32u * kEach;
    return c;
  }
};
// Q2_K: 16 scale bytes (low nibble scale, high nibble minimum, one a 16 values), 64 bytes of 2-bit codes, f16 d, f16
// dmin. Value 128 h + 32 r + l has its code at bits 2r of byte 16 + 32 h + l
template <> struct Layout<kQ2_K> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const int v0 = 8 * k, h = v0 >> 7, r = (v0 >> 5) & 3, l = v0 & 31;
    const uint8_t* q = b + 16 + 32 * h + l;
    const uint32_t s = b[v0 >> 4];
    return Chunk{{(ld32(q) >> (2 * r)) & 3u * kEach, (ld32(q + 4) >> (2 * r)) & 3u * kEach},
                 mul(half_at(b + 80), (float) (s & 15u)), mul(half_at(b + 82), (float) (s >> 4))};
  }
};
// Q3_K: 32 bytes of high bits, 64 bytes of 2-bit codes, 12 bytes of 6-bit scales, f16 d. Value 128 h + 32 r + l has its
// code at bits 2r of byte 32 + 32 h + l and its high bit at bit 4h + r of byte l; code = q2 + 4 hbit - 4. Scale s of
// the 16 sixteen-value groups (s = v / 16): low nibble from byte s % 8 (high nibble when s >= 8), top two bits at
// bits 2 (s / 4) of byte 8 + s % 4; the value is 6 bits - 32
template <> struct Layout<kQ3_K> {
  template <typename Tab> __device__ static Chunk at(const Tab&, const uint8_t* b, int k) {
    const int v0 = 8 * k, h = v0 >> 7, r = (v0 >> 5) & 3, l = v0 & 31, s = v0 >> 4;
    const uint8_t *q = b + 32 + 32 * h + l, *hm = b + l, *t = b + 96;
    const uint32_t sc = ((t[s & 7] >> (4 * (s >> 3))) & 15u) | ((t[8 + (s & 3)] >> (2 * (s >> 2))) & 3u) << 4;
    Chunk c{{0, 0}, mul(half_at(b + 108), (float) ((int) sc - 32)), 0.0f};
#pragma unroll
    for (int i = 0; i < 2; i++)
      c.w[i] = (((ld32(q + 4 * i) >> (2 * r)) & 3u * kEach) | ((ld32(hm + 4 * i) >> (4 * h + r)) & kEach) << 2) ^ 4u * kEach;
    return c;
  }
};
// IQ2_XXS: f16 d; a 32-group is 8 bytes: 4 grid indices (one a chunk) and a u32 of four 7-bit sign indices and a 4-bit
// scale s; value = ((d (0.5 + s)) / 4) * grid byte, signed
template <> struct Layout<kIQ2_XXS> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const uint8_t* g8 = b + 2 + 8 * (k >> 2);
    const uint32_t aux = ld32(g8 + 4);
    Chunk c{{0, 0}, mul(mul(half_at(b), 0.5f + (float) (aux >> 28)), 0.25f), 0.0f};
    signed_grid(c, K.g.iq2xxs[g8[k & 3]], ksign((aux >> (7 * (k & 3))) & 127u));
    return c;
  }
};
// IQ2_XS: f16 d, a u16 a chunk (9-bit grid index, 7-bit sign index), 8 scale bytes (a nibble a 16-value half group)
template <> struct Layout<kIQ2_XS> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const uint32_t e = ld16(b + 2 + 2 * k), s = (b[66 + (k >> 2)] >> (4 * ((k >> 1) & 1))) & 15u;
    Chunk c{{0, 0}, mul(mul(half_at(b), 0.5f + (float) s), 0.25f), 0.0f};
    signed_grid(c, K.g.iq2xs[e & 511u], ksign(e >> 9));
    return c;
  }
};
// IQ2_S: f16 d, 32 grid index low bytes, 32 sign bytes, 8 bytes of index high pairs, 8 scale bytes
template <> struct Layout<kIQ2_S> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const uint32_t s = (b[74 + (k >> 2)] >> (4 * ((k >> 1) & 1))) & 15u;
    const uint32_t idx = b[2 + k] | ((b[66 + (k >> 2)] >> (2 * (k & 3))) & 3u) << 8;
    Chunk c{{0, 0}, mul(mul(half_at(b), 0.5f + (float) s), 0.25f), 0.0f};
    signed_grid(c, K.g.iq2s[idx], b[34 + k]);
    return c;
  }
};
// IQ3_XXS: f16 d, 64 index bytes (one a 4 values into the 4-byte grid), then a u32 a 32-group (four 7-bit sign indices,
// scale s); value = ((d (0.5 + s)) / 2) * grid byte, signed
template <> struct Layout<kIQ3_XXS> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const uint8_t* idx = b + 2 + 2 * k;
    const uint32_t aux = ld32(b + 66 + 4 * (k >> 2));
    Chunk c{{0, 0}, mul(mul(half_at(b), 0.5f + (float) (aux >> 28)), 0.5f), 0.0f};
    signed_grid(c, (uint64_t) K.g.iq3xxs[idx[0]] | (uint64_t) K.g.iq3xxs[idx[1]] << 32,
                ksign((aux >> (7 * (k & 3))) & 127u));
    return c;
  }
};
// IQ1_S: f16 d, 32 grid index low bytes, a u16 a 32-group (3 index high bits a chunk, 3-bit s at bit 12, delta's sign
// at bit 15); value = (d (2s + 1)) * (grid + delta), delta +-1/8
template <> struct Layout<kIQ1_S> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    const uint32_t qh = ld16(b + 34 + 2 * (k >> 2));
    const uint64_t grid = K.g.iq1s[b[2 + k] | ((qh >> (3 * (k & 3))) & 7u) << 8];
    return Chunk{{(uint32_t) grid, (uint32_t) (grid >> 32)}, mul(half_at(b), (float) (2 * ((qh >> 12) & 7u) + 1)),
                 (qh >> 15) ? -0.125f : 0.125f};
  }
};
// IQ1_M: 32 grid index low bytes, 16 bytes of a nibble a chunk (3 index high bits, delta sign at bit 3), 8 bytes of
// 3-bit scales (one a 16 values, four to a u16) whose u16s' top nibbles together form the f16 d
template <> struct Layout<kIQ1_M> {
  template <typename Tab> __device__ static Chunk at(const Tab& K, const uint8_t* b, int k) {
    uint32_t dbits = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) dbits |= (ld16(b + 48 + 2 * i) >> 12) << (4 * i);
    const uint32_t s = (ld16(b + 48 + 2 * (k >> 3)) >> (3 * ((k >> 1) & 3))) & 7u;
    const uint32_t nib = (b[32 + (k >> 1)] >> (4 * (k & 1))) & 15u;
    const uint64_t grid = K.g.iq1s[b[k] | (nib & 7u) << 8];
    return Chunk{{(uint32_t) grid, (uint32_t) (grid >> 32)}, mul(f16(dbits), (float) (2 * s + 1)),
                 (nib & 8u) ? -0.125f : 0.125f};
  }
};

// the decoders: decode<T>(tables, block, chunk, values). `tables` is DecodeTables (the constant-memory codebooks) or
// any struct with the members the type reads (g.iq2xxs, iq4nl, ...) - mm.hip passes one held in LDS
template <uint32_t T, typename Tab> __device__ inline void decode(const Tab& K, const uint8_t* b, int k, float* v) {
  if constexpr (T == kF32) {
    const float4 a = *(const float4*) b, c = *(const float4*) (b + 16);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = c.x, v[5] = c.y, v[6] = c.z, v[7] = c.w;
  } else if constexpr (T == kBF16) {  // the top 16 bits of each fp32
    const uint4 a = *(const uint4*) b;
    const uint32_t p[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; i++) v[2 * i] = __uint_as_float(p[i] << 16), v[2 * i + 1] = __uint_as_float(p[i] & 0xFFFF0000u);
  } else {
    finish<T>(Layout<T>::at(K, b, k), v);
  }
}

// where a row's chunk c lies: its block and the chunk in it
template <uint32_t T>
__device__ inline const uint8_t* chunk_at(const uint8_t* row, uint32_t c, int* k) {
  constexpr uint32_t per = Block<T>::values / kChunk;
  *k = (int) (c % per);
  return row + (uint64_t) (c / per) * Block<T>::bytes;
}
// the same for any type with the row's index: its base (the row's start; Q5_KR's, its tile's) and, from it, the chunk
// (Q5_KR: the tile's block, chunk (row % 16) 32 + c % 32)
template <uint32_t T>
__device__ inline const uint8_t* row_base(const uint8_t* w, uint32_t row, uint32_t cols) {
  if constexpr (T == kQ5_KR) return w + (uint64_t) (row / 16) * 16 * row_bytes<T>(cols);
  else return w + (uint64_t) row * row_bytes<T>(cols);
}
template <uint32_t T>
__device__ inline const uint8_t* chunk_of(const uint8_t* base, uint32_t row, uint32_t c, int* k) {
  if constexpr (T == kQ5_KR) {
    *k = (int) ((row % 16) * 32 + c % 32);
    return base + (uint64_t) (c / 32) * 16 * Block<T>::bytes;
  } else {
    return chunk_at<T>(base, c, k);
  }
}

}  // namespace osm
