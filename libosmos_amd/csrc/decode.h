// libosmos MI355X - the GGUF blocks' exact fp32 values, 8 at a time (chunk k: values 8k .. 8k + 7 of a block), each
// the value gguf-py's dequantize gives: reference kernels/quant.h:60-348. products and subtracts are __fmul_rn /
// __fsub_rn (never contracted), so the bits are the reference's. shared by mv.hip (the fp32 matvec) and quant.hip.
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

__device__ inline float mul(float a, float b) { return __fmul_rn(a, b); }

// the decoders, one specialization a type: Dec<T>::run(tables, block, chunk, values). `tables` is DecodeTables (the
// constant-memory codebooks) or any struct with the members the type reads (g.iq2xxs, iq4nl, ...) - mm.hip passes
// one held in LDS. decode<T>(tables, ...) deduces the table's type
template <uint32_t T> struct Dec;
template <uint32_t T, typename Tab> __device__ inline void decode(const Tab& K, const uint8_t* b, int k, float* v) {
  Dec<T>::run(K, b, k, v);
}

template <> struct Dec<kF32> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int, float* v) {
    const float4 a = *(const float4*) b, c = *(const float4*) (b + 16);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = c.x, v[5] = c.y, v[6] = c.z, v[7] = c.w;
  }
};
template <> struct Dec<kBF16> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int, float* v) {
    const uint4 a = *(const uint4*) b;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; j++) v[2 * j] = __uint_as_float(w[j] << 16), v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
  }
};
// d * x (quant.h:66-69)
template <> struct Dec<kQ8_0> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const float d = f16(ld16(b));
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = mul((float) (int8_t) b[2 + k * kChunk + j], d);
  }
};
// d * (q - 8) (quant.h:242-248)
template <> struct Dec<kQ4_0> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const float d = f16(ld16(b));
    const uint32_t lo = ld32(b + 2 + (k % 2) * kChunk), hi = ld32(b + 6 + (k % 2) * kChunk);
    const int sh = 4 * (k / 2);
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = mul(d, (float) ((int) (((j < 4 ? lo : hi) >> (8 * (j % 4) + sh)) & 0x0F) - 8));
  }
};
// d * kvalues[q] (quant.h:199-205)
template <> struct Dec<kIQ4_NL> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const float d = f16(ld16(b));
    const uint8_t* qs = b + 2 + (k % 2) * kChunk;
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = mul(d, (float) K.iq4nl[(qs[j] >> (4 * (k / 2))) & 0x0F]);
  }
};

__device__ inline void k_scale_min(const uint8_t* s, int g, int& sc, int& m) {
  sc = g < 4 ? s[g] & 0x3F : (s[g + 4] & 0x0F) | ((s[g - 4] >> 2) & 0x30);
  m = g < 4 ? s[g + 4] & 0x3F : (s[g + 4] >> 4) | ((s[g] >> 2) & 0x30);
}
// (d * sc) * q - (dmin * m) (quant.h:89-103)
template <> struct Dec<kQ4_K> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const int g = k / 4, l0 = (k % 4) * kChunk;
    int sc, m;
    k_scale_min(b + 4, g, sc, m);
    const float d = mul(f16(ld16(b)), (float) sc), dm = mul(f16(ld16(b + 2)), (float) m);
    const uint8_t* qs = b + 16 + (g / 2) * 32 + l0;
    const uint32_t q0 = ld32(qs), q1 = ld32(qs + 4);
    const int sh = 4 * (g % 2);
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = __fsub_rn(mul(d, (float) (((j < 4 ? q0 : q1) >> (8 * (j % 4) + sh)) & 0x0F)), dm);
  }
};
// (quant.h:71-87)
template <> struct Dec<kQ5_K> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const int g = k / 4, l0 = (k % 4) * kChunk;
    int sc, m;
    k_scale_min(b + 4, g, sc, m);
    const float d = mul(f16(ld16(b)), (float) sc), dm = mul(f16(ld16(b + 2)), (float) m);
    const uint8_t *qh = b + 16 + l0, *qs = b + 48 + (g / 2) * 32 + l0;
#pragma unroll
    for (int j = 0; j < kChunk; j++) {
      const int q = ((qs[j] >> (4 * (g % 2))) & 0x0F) | (((qh[j] >> g) & 1) << 4);
      v[j] = __fsub_rn(mul(d, (float) q), dm);
    }
  }
};
// (d * sc) * (q - 32) (quant.h:164-179)
template <> struct Dec<kQ6_K> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t* sc = (const int8_t*) (b + 192);
    const float d0 = f16(ld16(b + 208));
    const int g = k / 4, h = g / 4, r = g % 4, l0 = (k % 4) * kChunk;
    const float d = mul(d0, (float) sc[(g * 32 + l0) / 16]);
#pragma unroll
    for (int j = 0; j < kChunk; j++) {
      const int l = l0 + j;
      const int lo = (ql[h * 64 + (r % 2) * 32 + l] >> (4 * (r / 2))) & 0x0F;
      const int hi = (qh[h * 32 + l] >> (2 * r)) & 0x03;
      v[j] = mul(d, (float) ((lo | hi << 4) - 32));
    }
  }
};
// (quant.h:250-262)
template <> struct Dec<kQ2_K> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const int g = k / 2, l0 = (k % 4) * kChunk, shift = 2 * ((k % 16) / 4);
    const uint8_t* qs = b + 16 + 32 * (k / 16) + l0;
    const float dl = mul(f16(ld16(b + 80)), (float) (b[g] & 0x0F));
    const float ml = mul(f16(ld16(b + 82)), (float) (b[g] >> 4));
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = __fsub_rn(mul(dl, (float) ((qs[j] >> shift) & 0x03)), ml);
  }
};
// (quant.h:264-284)
template <> struct Dec<kQ3_K> {
  template <typename Tab> __device__ static inline void run(const Tab&, const uint8_t* b, int k, float* v) {
    const int i0 = k * kChunk, n = i0 / 128, r = i0 % 128, j = r / 32, sub = (r % 32) / 16, l0 = r % 16;
    const int g = 8 * n + 2 * j + sub, grp = g / 4, w = g % 4;
    const uint8_t* sc = b + 96;
    const int low = ((grp & 1 ? sc[4 + w] : sc[w]) >> (grp & 2 ? 4 : 0)) & 0x0F;
    const int sc6 = low | ((sc[8 + w] >> (2 * grp)) & 0x03) << 4;
    const float dl = mul(f16(ld16(b + 108)), (float) (sc6 - 32));
    const uint8_t *qs = b + 32 + 32 * n + 16 * sub + l0, *hm = b + 16 * sub + l0;
    const int bit = 4 * n + j;
#pragma unroll
    for (int jj = 0; jj < kChunk; jj++) v[jj] = mul(dl, (float) (((qs[jj] >> (2 * j)) & 0x03) - ((hm[jj] >> bit) & 1 ? 0 : 4)));
  }
};

__device__ inline void sgn8(float db, uint64_t grid, uint32_t signs, float* v) {
#pragma unroll
  for (int j = 0; j < kChunk; j++) {
    const float x = mul(db, (float) (uint8_t) (grid >> (8 * j)));
    v[j] = (signs >> j) & 1 ? -x : x;
  }
}
// ((d * (0.5 + s)) * 0.25) * grid, signed (quant.h:181-197)
template <> struct Dec<kIQ2_XXS> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const uint8_t* q = b + 2 + (k / 4) * 8;
    const uint32_t aux = ld32(q + 4);
    const float db = mul(mul(f16(ld16(b)), 0.5f + (float) (aux >> 28)), 0.25f);
    sgn8(db, K.g.iq2xxs[q[k % 4]], ksign((aux >> (7 * (k % 4))) & 0x7F), v);
  }
};
template <> struct Dec<kIQ2_XS> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const uint32_t q = ld16(b + 2 + 2 * k);
    const int s = (b[66 + k / 4] >> (4 * ((k / 2) % 2))) & 0x0F;
    const float db = mul(mul(f16(ld16(b)), 0.5f + (float) s), 0.25f);
    sgn8(db, K.g.iq2xs[q & 511], ksign(q >> 9), v);
  }
};
template <> struct Dec<kIQ2_S> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const int s = (b[74 + k / 4] >> (4 * ((k / 2) % 2))) & 0x0F;
    const float db = mul(mul(f16(ld16(b)), 0.5f + (float) s), 0.25f);
    sgn8(db, K.g.iq2s[b[2 + k] | ((b[66 + k / 4] >> (2 * (k % 4))) & 0x03) << 8], b[34 + k], v);
  }
};
// ((d * (0.5 + s)) * 0.5) * grid, signed (quant.h:217-230)
template <> struct Dec<kIQ3_XXS> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const uint8_t* q = b + 2 + (k / 4) * 8 + (k % 4) * 2;
    const uint32_t aux = ld32(b + 2 + 64 + (k / 4) * 4);
    const float db = mul(mul(f16(ld16(b)), 0.5f + (float) (aux >> 28)), 0.5f);
    const uint64_t grid = (uint64_t) K.g.iq3xxs[q[0]] | (uint64_t) K.g.iq3xxs[q[1]] << 32;
    sgn8(db, grid, ksign((aux >> (7 * (k % 4))) & 0x7F), v);
  }
};
// (quant.h:232-240)
template <> struct Dec<kIQ4_XS> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const int g = k / 4, j0 = (k % 4) * kChunk;
    const int ls = ((b[4 + g / 2] >> (4 * (g % 2))) & 0x0F) | ((ld16(b + 2) >> (2 * g)) & 0x03) << 4;
    const float dl = mul(f16(ld16(b)), (float) (ls - 32));
    const uint8_t* qs = b + 8 + 16 * g + j0 % 16;
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = mul(dl, (float) K.iq4nl[(qs[j] >> (4 * (j0 / 16))) & 0x0F]);
  }
};
// (d * (2s + 1)) * (grid + delta) (quant.h:313-336)
template <> struct Dec<kIQ1_S> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const uint32_t h = ld16(b + 34 + 2 * (k / 4));
    const float dl = mul(f16(ld16(b)), (float) (2 * ((h >> 12) & 0x07) + 1));
    const float delta = h & 0x8000 ? -0.125f : 0.125f;
    const uint64_t grid = K.g.iq1s[b[2 + k] | ((h >> (3 * (k % 4))) & 0x07) << 8];
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = mul(dl, __fadd_rn((float) (int8_t) (grid >> (8 * j)), delta));
  }
};
template <> struct Dec<kIQ1_M> {
  template <typename Tab> __device__ static inline void run(const Tab& K, const uint8_t* b, int k, float* v) {
    const uint32_t sc0 = ld32(b + 48), sc1 = ld32(b + 52);
    const uint64_t sc = (uint64_t) sc0 | (uint64_t) sc1 << 32;
    const uint32_t s0 = sc0 & 0xFFFF, s1 = sc0 >> 16, s2 = sc1 & 0xFFFF, s3 = sc1 >> 16;
    const float d = f16((s0 >> 12) | ((s1 >> 8) & 0x00F0) | ((s2 >> 4) & 0x0F00) | (s3 & 0xF000));
    const int s = (int) ((sc >> (16 * (k / 8) + 3 * ((k / 2) % 4))) & 0x07);
    const float dl = mul(d, (float) (2 * s + 1));
    const uint32_t h = (b[32 + k / 2] >> (4 * (k % 2))) & 0x0F;
    const float delta = h & 0x08 ? -0.125f : 0.125f;
    const uint64_t grid = K.g.iq1s[b[k] | (h & 0x07) << 8];
#pragma unroll
    for (int j = 0; j < kChunk; j++) v[j] = mul(dl, __fadd_rn((float) (int8_t) (grid >> (8 * j)), delta));
  }
};

// where a row's chunk c lies (reference kernels/quant.h:124-150): its block and the chunk in it
template <uint32_t T>
__device__ inline const uint8_t* chunk_at(const uint8_t* row, uint32_t c, int* k) {
  constexpr uint32_t per = Block<T>::values / kChunk;
  *k = (int) (c % per);
  return row + (uint64_t) (c / per) * Block<T>::bytes;
}

}  // namespace osm
