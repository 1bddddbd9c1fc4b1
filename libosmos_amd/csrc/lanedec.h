// libosmos MI355X - the lane contract's per-block arithmetic, shared by the lane kernels (lane.hip) and the fused
// layer kernels (layer.hip): each type's 32-value block as int8 codes and scale integers (reference kernels/q8.h:28-130,
// and this build's Q4_0 / Q4_K / Q3_K codes), the block's exact integer half-dots and the contract's float steps
// (reference kernels/q8.h:133-162, kernels/lane.h:54-68), the lane tree, the input-row rule (kernels/q8.h:164-173).
#pragma once
#include "common.h"

namespace osm {
namespace lane {

static __constant__ Grids kGrids = make_grids();

// IQ3_XXS's codebook with its signs applied: entry 16 g + s is grid entry g's 4 values (bytes 4..62), value i negated
// where bit i of s is set, as 4 int8 in a word - a block's 8 words are then 8 lookups, no per-value sign arithmetic
struct alignas(16) SignedIq3 {
  uint32_t v[256 * 16];
};
constexpr SignedIq3 make_signed_iq3() {
  const Grids g = make_grids();
  SignedIq3 t{};
  for (int e = 0; e < 256; e++)
    for (int sg = 0; sg < 16; sg++) {
      uint32_t w = 0;
      for (int i = 0; i < 4; i++) {
        const int v = (int) ((g.iq3xxs[e] >> (8 * i)) & 0xFF);
        w |= (uint32_t) (uint8_t) (int8_t) ((sg >> i) & 1 ? -v : v) << (8 * i);
      }
      t.v[16 * e + sg] = w;
    }
  return t;
}
static __constant__ SignedIq3 kSignedIq3 = make_signed_iq3();

// a 32-value block's int8 codes: 8 words (4 values each, value 4i + b in byte b of word i); per 8-value chunk k the
// IQ1 types' delta (+-1, codes 8 grid + delta) or 0; per 16-value half its scale integer s21 (Q2_K, Q4_K: 8 sc) and
// minimum m8 (8 m); the block scale d and minimum scale dmin. `bias`: a constant subtracted from every code (Q4_0's
// 8, Q3_K's 4), applied to the integer dot through x's sum - the same integer
struct Codes {
  int w[8];
  int delta[4];
  int s21[2];
  int m8[2];
  float d, dmin;
};

// 8 unsigned grid bytes, each negated where its sign bit is set: (v ^ m) + (m & 1) a byte, m = 0xFF where negative
__device__ inline void signed8(uint64_t grid, uint32_t signs, int& lo, int& hi) {
  uint32_t a = 0, b = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a |= ((signs >> i) & 1u) * (0xFFu << (8 * i));
    b |= ((signs >> (4 + i)) & 1u) * (0xFFu << (8 * i));
  }
  lo = (int) (((uint32_t) grid ^ a) + (a & 0x01010101u));
  hi = (int) (((uint32_t) (grid >> 32) ^ b) + (b & 0x01010101u));
}

__device__ inline int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <uint32_t T> struct Traits {
  static constexpr bool iq1 = false, has_min = false, whole = false;
  static constexpr int bias = 0;  // subtracted from each code
};
template <> struct Traits<kIQ1_M> { static constexpr bool iq1 = true, has_min = false, whole = false; static constexpr int bias = 0; };
template <> struct Traits<kIQ1_S> { static constexpr bool iq1 = true, has_min = false, whole = false; static constexpr int bias = 0; };
template <> struct Traits<kQ2_K> { static constexpr bool iq1 = false, has_min = true, whole = false; static constexpr int bias = 0; };
template <> struct Traits<kQ4_0> { static constexpr bool iq1 = false, has_min = false, whole = true; static constexpr int bias = 8; };
template <> struct Traits<kQ4_K> { static constexpr bool iq1 = false, has_min = true, whole = true; static constexpr int bias = 0; };
template <> struct Traits<kQ3_K> { static constexpr bool iq1 = false, has_min = false, whole = false; static constexpr int bias = 4; };

// each codebook type's table: its element type and length; `G` below is a pointer to it (constant memory or a
// workgroup's LDS copy)
template <uint32_t T> struct GridOf { using E = uint8_t; static constexpr int n = 0; };
template <> struct GridOf<kIQ2_XXS> { using E = uint64_t; static constexpr int n = 256; };
template <> struct GridOf<kIQ2_XS> { using E = uint64_t; static constexpr int n = 512; };
template <> struct GridOf<kIQ2_S> { using E = uint64_t; static constexpr int n = 1024; };
template <> struct GridOf<kIQ1_S> { using E = uint64_t; static constexpr int n = 2048; };
template <> struct GridOf<kIQ1_M> { using E = uint64_t; static constexpr int n = 2048; };
template <> struct GridOf<kIQ3_XXS> { using E = uint32_t; static constexpr int n = 256 * 16; };  // signed

template <uint32_t T> __device__ inline const typename GridOf<T>::E* const_grid() {
  if constexpr (T == kIQ2_XXS) return kGrids.iq2xxs;
  else if constexpr (T == kIQ2_XS) return kGrids.iq2xs;
  else if constexpr (T == kIQ2_S) return kGrids.iq2s;
  else if constexpr (T == kIQ1_S || T == kIQ1_M) return kGrids.iq1s;
  else if constexpr (T == kIQ3_XXS) return kSignedIq3.v;
  else return nullptr;
}

// the block bytes' readers: from generic (global) memory, or from LDS (lbytes: an LDS address). a 2-aligned address's
// 16-bit words are read one at a time in LDS (ld16s: volatile, so the compiler does not merge neighbours into one
// wider read, which LDS serves slowly when the address is not aligned to its width); elsewhere plain reads
typedef const __attribute__((address_space(3))) uint8_t* lbytes;
typedef const __attribute__((address_space(3))) volatile uint16_t* lds16v;
using osm::ld16;
__device__ inline uint32_t ld16(lbytes p) { return *(const __attribute__((address_space(3))) uint16_t*) p; }
__device__ inline uint32_t ld16s(const uint8_t* p) { return ld16(p); }
__device__ inline uint32_t ld16s(lbytes p) { return *(lds16v) p; }
template <typename B> __device__ inline uint32_t ld32s(B p) { return ld16s(p) | ld16s(p + 2) << 16; }
template <typename B> __device__ inline uint32_t ld32b(B p) { return ld16(p) | ld16(p + 2) << 16; }

// reference kernels/q8.h:46-55
template <typename B> __device__ inline void codes_kIQ2_XXS(B b, int j, Codes& c, const GridOf<kIQ2_XXS>::E* grid) {
  const auto q = b + 2 + 8 * j;
  const uint32_t qi = ld32s(q), aux = ld32s(q + 4);
#pragma unroll
  for (int k = 0; k < 4; k++)
    signed8(grid[(qi >> (8 * k)) & 0xFF], ksign((aux >> (7 * k)) & 0x7F), c.w[2 * k], c.w[2 * k + 1]);
  c.s21[0] = c.s21[1] = 2 * (int) (aux >> 28) + 1;
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:57-66
template <typename B> __device__ inline void codes_kIQ2_XS(B b, int j, Codes& c, const GridOf<kIQ2_XS>::E* grid) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t q = ld16s(b + 2 + 2 * (4 * j + k));
    signed8(grid[q & 511], ksign(q >> 9), c.w[2 * k], c.w[2 * k + 1]);
  }
  const uint32_t s = b[66 + j];
  c.s21[0] = 2 * (int) (s & 0x0F) + 1, c.s21[1] = 2 * (int) (s >> 4) + 1;
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:68-84
template <typename B> __device__ inline void codes_kIQ1_M(B b, int j, Codes& c, const GridOf<kIQ1_M>::E* grid) {
  const uint32_t sc0 = ld32b(b + 48), sc1 = ld32b(b + 52);
  const uint64_t sc = (uint64_t) sc0 | (uint64_t) sc1 << 32;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int kk = 4 * j + k;
    const uint32_t h = (b[32 + kk / 2] >> (4 * (kk % 2))) & 0x0F;
    const uint64_t g = grid[b[kk] | (h & 0x07) << 8];
    c.w[2 * k] = (int) (uint32_t) g, c.w[2 * k + 1] = (int) (uint32_t) (g >> 32);
    c.delta[k] = h & 0x08 ? -1 : 1;
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int kk = 4 * j + 2 * h;
    c.s21[h] = 2 * (int) ((sc >> (16 * (kk / 8) + 3 * ((kk / 2) % 4))) & 0x07) + 1;
  }
  const uint32_t s0 = sc0 & 0xFFFF, s1 = sc0 >> 16, s2 = sc1 & 0xFFFF, s3 = sc1 >> 16;
  c.d = f16((s0 >> 12) | ((s1 >> 8) & 0x00F0) | ((s2 >> 4) & 0x0F00) | (s3 & 0xF000));
}

// reference kernels/q8.h:86-95
template <typename B> __device__ inline void codes_kIQ2_S(B b, int j, Codes& c, const GridOf<kIQ2_S>::E* grid) {
  const uint32_t qi = ld32s(b + 2 + 4 * j), sg = ld32s(b + 34 + 4 * j), hi = b[66 + j];
#pragma unroll
  for (int k = 0; k < 4; k++)
    signed8(grid[((qi >> (8 * k)) & 0xFF) | ((hi >> (2 * k)) & 0x03) << 8], (sg >> (8 * k)) & 0xFF, c.w[2 * k],
            c.w[2 * k + 1]);
  const uint32_t s = b[74 + j];
  c.s21[0] = 2 * (int) (s & 0x0F) + 1, c.s21[1] = 2 * (int) (s >> 4) + 1;
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:97-108 (the same codes: grid entries q[2k] and q[2k + 1] signed by ksign's 8 bits - its low
// nibble the first entry's, its top 3 bits and the 7-bit index's parity the second's), read from the signed table;
// the four 7-bit fields' parities at once: y folds x over 8 bits, so bit 7k of y ^ (x >> 7) is field k's parity
template <typename B> __device__ inline void codes_kIQ3_XXS(B b, int j, Codes& c, const GridOf<kIQ3_XXS>::E* grid) {
  const auto q = b + 2 + 8 * j;
  const uint32_t q03 = ld32s(q), q47 = ld32s(q + 4);
  const uint32_t aux = ld32s(b + 66 + 4 * j);
  const uint32_t x = aux & 0x0FFFFFFFu;
  uint32_t y = x ^ (x >> 1);
  y ^= y >> 2;
  y ^= y >> 4;
  const uint32_t par = y ^ (x >> 7);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t sg = (aux >> (7 * k)) & 0x7F, qq = k < 2 ? q03 : q47;
    const uint32_t g0 = (qq >> (16 * (k % 2))) & 0xFF, g1 = (qq >> (16 * (k % 2) + 8)) & 0xFF;
    c.w[2 * k] = (int) grid[16 * g0 + (sg & 15)];
    c.w[2 * k + 1] = (int) grid[16 * g1 + ((sg >> 4) | ((par >> (7 * k)) & 1) << 3)];
  }
  c.s21[0] = c.s21[1] = 2 * (2 * (int) (aux >> 28) + 1);
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:110-118
template <typename B> __device__ inline void codes_kQ2_K(B b, int j, Codes& c, const GridOf<kQ2_K>::E* grid) {
  const auto qs = b + 16 + 32 * (j / 4);
  const int shift = 2 * (j % 4);
#pragma unroll
  for (int t = 0; t < 8; t++) c.w[t] = (int) ((ld32b(qs + 4 * t) >> shift) & 0x03030303u);
#pragma unroll
  for (int h = 0; h < 2; h++) c.s21[h] = 8 * (b[2 * j + h] & 0x0F), c.m8[h] = 8 * (b[2 * j + h] >> 4);
  c.d = f16(ld16(b + 80)), c.dmin = f16(ld16(b + 82));
}

// reference kernels/q8.h:120-130
template <typename B> __device__ inline void codes_kIQ1_S(B b, int j, Codes& c, const GridOf<kIQ1_S>::E* grid) {
  const uint32_t h = ld16(b + 34 + 2 * j), qi = ld32s(b + 2 + 4 * j);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint64_t g = grid[((qi >> (8 * k)) & 0xFF) | ((h >> (3 * k)) & 0x07) << 8];
    c.w[2 * k] = (int) (uint32_t) g, c.w[2 * k + 1] = (int) (uint32_t) (g >> 32);
    c.delta[k] = h & 0x8000 ? -1 : 1;
  }
  c.s21[0] = c.s21[1] = 2 * (int) ((h >> 12) & 0x07) + 1;
  c.d = f16(ld16(b));
}

// build-defined: ggml's Q4_0 (32 values: f16 d, 16 bytes of nibbles; value i < 16 byte i's low nibble, 16 + i its
// high), codes q - 8 (the 8 through `bias`), one part over the 32 with s21 8 - so d * isum exactly
template <typename B> __device__ inline void codes_kQ4_0(B b, int, Codes& c, const GridOf<kQ4_0>::E* grid) {
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const uint32_t v = ld32s(b + 2 + 4 * t);
    c.w[t] = (int) (v & 0x0F0F0F0Fu), c.w[4 + t] = (int) ((v >> 4) & 0x0F0F0F0Fu);
  }
  c.s21[0] = c.s21[1] = 8;
  c.d = f16(ld16(b));
}

// build-defined: Q4_K's group j (its 6-bit sc and m, reference kernels/quant.h:89-103's layout), codes q, one part
// with its minimum: ((d * 8 sc) / 8) * isum - ((dmin * 8 m) / 8) * xsum
template <typename B> __device__ inline void codes_kQ4_K(B b, int j, Codes& c, const GridOf<kQ4_K>::E* grid) {
  const auto s = b + 4;
  const int sc = j < 4 ? s[j] & 0x3F : (s[j + 4] & 0x0F) | ((s[j - 4] >> 2) & 0x30);
  const int m = j < 4 ? s[j + 4] & 0x3F : (s[j + 4] >> 4) | ((s[j] >> 2) & 0x30);
  const auto qs = b + 16 + (j / 2) * 32;
  const int sh = 4 * (j % 2);
#pragma unroll
  for (int t = 0; t < 8; t++) c.w[t] = (int) ((ld32b(qs + 4 * t) >> sh) & 0x0F0F0F0Fu);
  c.s21[0] = c.s21[1] = 8 * sc, c.m8[0] = c.m8[1] = 8 * m;
  c.d = f16(ld16(b)), c.dmin = f16(ld16(b + 2));
}

// build-defined: Q3_K's values 32 j .. 32 j + 31 (reference kernels/quant.h:264-284's layout): codes q2 + 4 h - 4
// (the 4 through `bias`), two halves, each s21 = 8 (sc - 32) of its 16-value group
template <typename B> __device__ inline void codes_kQ3_K(B b, int j, Codes& c, const GridOf<kQ3_K>::E* grid) {
  const int n = j / 4, jj = j % 4;
  const auto qs = b + 32 + 32 * n;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    const uint32_t q2 = (ld32b(qs + 4 * t) >> (2 * jj)) & 0x03030303u;
    const uint32_t hb = (ld32b(b + 4 * t) >> (4 * n + jj)) & 0x01010101u;
    c.w[t] = (int) (q2 + (hb << 2));
  }
  const auto sc = b + 96;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int g = 2 * j + h, grp = g / 4, w = g % 4;
    const int low = ((grp & 1 ? sc[4 + w] : sc[w]) >> (grp & 2 ? 4 : 0)) & 0x0F;
    const int sc6 = low | ((sc[8 + w] >> (2 * grp)) & 0x03) << 4;
    c.s21[h] = 8 * (sc6 - 32);
  }
  c.d = f16(ld16(b + 108));
}

template <uint32_t T, typename B>
__device__ __forceinline__ void codes(B b, int j, Codes& c, const typename GridOf<T>::E* grid) {
  if constexpr (T == kIQ2_XXS) codes_kIQ2_XXS(b, j, c, grid);
  else if constexpr (T == kIQ2_XS) codes_kIQ2_XS(b, j, c, grid);
  else if constexpr (T == kIQ1_M) codes_kIQ1_M(b, j, c, grid);
  else if constexpr (T == kIQ2_S) codes_kIQ2_S(b, j, c, grid);
  else if constexpr (T == kIQ3_XXS) codes_kIQ3_XXS(b, j, c, grid);
  else if constexpr (T == kQ2_K) codes_kQ2_K(b, j, c, grid);
  else if constexpr (T == kIQ1_S) codes_kIQ1_S(b, j, c, grid);
  else if constexpr (T == kQ4_0) codes_kQ4_0(b, j, c, grid);
  else if constexpr (T == kQ4_K) codes_kQ4_K(b, j, c, grid);
  else if constexpr (T == kQ3_K) codes_kQ3_K(b, j, c, grid);
}

// the block's contribution before x's scale (reference kernels/q8.h:133-162)
template <uint32_t T>
__device__ inline float block_sum(const Codes& c, const int* x) {
  using Tr = Traits<T>;
  int isum[2], xsum[2];
  if constexpr (!Tr::iq1 && !Tr::has_min && !Tr::bias) {  // a half's 4 dots in one chain (the same integer)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int s = 0;
#pragma unroll
      for (int i = 4 * h; i < 4 * h + 4; i++) s = dot4(c.w[i], x[i], s);
      isum[h] = s, xsum[h] = 0;
    }
  } else
#pragma unroll
  for (int h = 0; h < 2; h++) {
    int s = 0, sx = 0;
#pragma unroll
    for (int k = 2 * h; k < 2 * h + 2; k++) {
      const int gx = dot4(c.w[2 * k + 1], x[2 * k + 1], dot4(c.w[2 * k], x[2 * k], 0));
      if constexpr (Tr::iq1 || Tr::has_min || Tr::bias) {
        const int xk = dot4(0x01010101, x[2 * k + 1], dot4(0x01010101, x[2 * k], 0));
        if constexpr (Tr::iq1) s += 8 * gx + c.delta[k] * xk;
        else s += gx - Tr::bias * xk;
        sx += xk;
      } else {
        s += gx;
      }
    }
    isum[h] = s, xsum[h] = sx;
  }
  if constexpr (Tr::whole) {
    const int is = isum[0] + isum[1];
    if constexpr (Tr::has_min)
      return __fsub_rn(lane_part(c.d, c.s21[0], is), lane_part(c.dmin, c.m8[0], xsum[0] + xsum[1]));
    else
      return lane_part(c.d, c.s21[0], is);
  } else if constexpr (Tr::has_min) {
    const float p0 = __fsub_rn(lane_part(c.d, c.s21[0], isum[0]), lane_part(c.dmin, c.m8[0], xsum[0]));
    const float p1 = __fsub_rn(lane_part(c.d, c.s21[1], isum[1]), lane_part(c.dmin, c.m8[1], xsum[1]));
    return __fadd_rn(p0, p1);
  } else {
    return __fadd_rn(lane_part(c.d, c.s21[0], isum[0]), lane_part(c.d, c.s21[1], isum[1]));
  }
}

// a launch's NT input rows for output rows r0 .. r0 + NT - 1 (reference kernels/q8.h:164-173): row r's own (xin
// NULL), else row xin[r]; the rows past the count read as the count's last - summed, never stored
template <int NT>
__device__ inline void in_rows(const int32_t* xin, uint32_t r0, uint32_t cnt, uint64_t* xr) {
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const uint32_t r = r0 + ((uint32_t) t < cnt ? (uint32_t) t : cnt - 1);
    xr[t] = xin ? (uint64_t) (uint32_t) xin[r] : r;
  }
}

__device__ inline void load_x(const int8_t* q, uint64_t at, int* x) {
  const int4* xp = (const int4*) (q + at);
  const int4 a = xp[0], b = xp[1];
  x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
}

// the lanes' xor tree over the row's L logical lanes: acc[l] + acc[l ^ o], o = L/2 .. 1 (reference kernels/q8.h:209)
template <int L>
__device__ inline float tree(float v) {
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) v = __fadd_rn(v, xor_lane(v, o));
  return v;
}


}  // namespace lane
}  // namespace osm
