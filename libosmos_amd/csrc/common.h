// libosmos MI355X - device-side foundations shared by every kernel file: the GGUF block table, the codebooks (expanded
// at compile time from iq_grids.h into constant memory), byte loads that tolerate the formats' 2-byte alignment, and
// the lane contract's float helpers (reference kernels/lane.h:17-75). gfx950 (CDNA4), wave64.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "iq_grids.h"

// the library's exports: everything else is hidden (built -fvisibility=hidden)
#define OSM_API __attribute__((visibility("default")))

namespace osm {

constexpr int kWave = 64;  // CDNA: a wavefront is 64 lanes

// GGUF type ids (reference include/osmos/model/qtype.h:28-53)
enum Type : uint32_t {
  kF32 = 0, kQ4_0 = 2, kQ8_0 = 8, kQ2_K = 10, kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kIQ2_XXS = 16,
  kIQ2_XS = 17, kIQ3_XXS = 18, kIQ1_S = 19, kIQ4_NL = 20, kIQ2_S = 22, kIQ4_XS = 23, kIQ1_M = 29, kBF16 = 30,
  kQ5_KR = 0x100 | 13,  // Q5_K repacked in tiles of 16 rows (reference include/osmos/gpu/quant.h:17: QUANT_Q5_KR)
};

template <uint32_t T> struct Block;
#define OSM_BLOCK(t, v, b) \
  template <> struct Block<t> { static constexpr uint32_t values = v, bytes = b; };
OSM_BLOCK(kF32, 8, 32)    // fp32 and bf16: a "block" is one chunk of 8 values
OSM_BLOCK(kBF16, 8, 16)
OSM_BLOCK(kQ4_0, 32, 18)
OSM_BLOCK(kQ8_0, 32, 34)
OSM_BLOCK(kIQ4_NL, 32, 18)
OSM_BLOCK(kQ2_K, 256, 84)
OSM_BLOCK(kQ3_K, 256, 110)
OSM_BLOCK(kQ4_K, 256, 144)
OSM_BLOCK(kQ5_K, 256, 176)
OSM_BLOCK(kQ5_KR, 256, 180)  // (a row's share of its tile's block: 16 rows x 180 bytes a block of 256 columns)
OSM_BLOCK(kQ6_K, 256, 210)
OSM_BLOCK(kIQ2_XXS, 256, 66)
OSM_BLOCK(kIQ2_XS, 256, 74)
OSM_BLOCK(kIQ3_XXS, 256, 98)
OSM_BLOCK(kIQ1_S, 256, 50)
OSM_BLOCK(kIQ2_S, 256, 82)
OSM_BLOCK(kIQ4_XS, 256, 136)
OSM_BLOCK(kIQ1_M, 256, 56)
#undef OSM_BLOCK

template <uint32_t T> constexpr uint64_t row_bytes(uint32_t cols) {
  return (uint64_t) (cols / Block<T>::values) * Block<T>::bytes;
}

// ---- the codebooks: expanded from the packed index lists at compile time, one constant-memory table a grid ----
struct alignas(16) Grids {
  uint64_t iq2xxs[256];
  uint64_t iq2xs[512];
  uint64_t iq2s[1024];
  uint64_t iq1s[2048];
  uint32_t iq3xxs[256];
};

constexpr uint64_t expand8(uint16_t p, uint8_t m0, uint8_t m1, uint8_t m2) {
  uint64_t r = 0;
  for (int i = 0; i < 8; i++) {
    const int k = (p >> (2 * i)) & 3;
    r |= (uint64_t) (k == 0 ? m0 : k == 1 ? m1 : m2) << (8 * i);
  }
  return r;
}

constexpr Grids make_grids() {
  constexpr uint16_t p2xxs[] = {IQ_PACKED_IQ2XXS};
  constexpr uint16_t p2xs[] = {IQ_PACKED_IQ2XS};
  constexpr uint16_t p2s[] = {IQ_PACKED_IQ2S};
  constexpr uint16_t p1s[] = {IQ_PACKED_IQ1S};
  constexpr uint16_t p3xxs[] = {IQ_PACKED_IQ3XXS};
  constexpr uint8_t m3[8] = {0x04, 0x0c, 0x14, 0x1c, 0x24, 0x2c, 0x34, 0x3e};
  Grids g{};
  for (int i = 0; i < 256; i++) g.iq2xxs[i] = expand8(p2xxs[i], 0x08, 0x19, 0x2b);
  for (int i = 0; i < 512; i++) g.iq2xs[i] = expand8(p2xs[i], 0x08, 0x19, 0x2b);
  for (int i = 0; i < 1024; i++) g.iq2s[i] = expand8(p2s[i], 0x08, 0x19, 0x2b);
  for (int i = 0; i < 2048; i++) g.iq1s[i] = expand8(p1s[i], 0xff, 0x00, 0x01);
  for (int i = 0; i < 256; i++) {
    uint32_t r = 0;
    for (int k = 0; k < 4; k++) r |= (uint32_t) m3[(p3xxs[i] >> (3 * k)) & 7] << (8 * k);
    g.iq3xxs[i] = r;
  }
  return g;
}

// ---- loads: GGUF blocks are 2-byte aligned (their sizes are even), so wider words come from aligned dwords ----
__device__ inline uint32_t ld8(const uint8_t* p) { return *p; }
__device__ inline uint32_t ld16(const uint8_t* p) { return *(const uint16_t*) p; }
// a load through the global address space: a pointer the compiler cannot place (one read from a table, a struct's)
// would otherwise be a flat load, which also counts against the LDS wait counter - every wait for an LDS read would
// then wait for it too
// entry i of a device table of pointers to global memory (weight matrices' tables), read as a global-space pointer:
// every load derived from it is then a global load, where a pointer read as a generic one makes flat loads (which
// also count against the LDS wait counter, so each wait for an LDS read would wait for them too)
template <typename T>
__device__ inline T* table_at(T* const* tab, uint32_t i) {
  typedef __attribute__((address_space(1))) T* G;
  const G g = ((const G*) tab)[i];
  return (T*) g;
}
template <typename V>
__device__ inline V gload(const void* p) {
  return *(const __attribute__((address_space(1))) V*) p;
}
__device__ inline uint32_t ld32(const uint8_t* p) { return ld16(p) | ld16(p + 2) << 16; }
__device__ inline float f16(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short) bits)); }

// a 7-bit sign index as 8 signs, bit 7 its parity (gguf's ksigns table, computed)
__device__ inline uint32_t ksign(uint32_t i) { return i | ((__builtin_popcount(i) & 1u) << 7); }

// ---- cross-lane: the value of lane (this lane ^ o), o in 1 .. 16, within the lane's aligned group of 32 (DPP
// quad permutes for 1 and 2, ds_swizzle's xor mode for 4 .. 16): the exact xor partner a tree needs ----
__device__ inline int xor_lane(int x, int o) {
  if (o == 1) return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
  if (o == 2) return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
  switch (o) {  // bitmask mode: source lane = (lane & 31) ^ o
    case 4: return __builtin_amdgcn_ds_swizzle(x, (4 << 10) | 0x1F);
    case 8: return __builtin_amdgcn_ds_swizzle(x, (8 << 10) | 0x1F);
    default: return __builtin_amdgcn_ds_swizzle(x, (16 << 10) | 0x1F);
  }
}
__device__ inline float xor_lane(float v, int o) { return __int_as_float(xor_lane(__float_as_int(v), o)); }

// ---- the lane contract's float helpers (reference kernels/lane.h:17-75) ----
__device__ inline float lane_exp(float x) {
  if (x > 88.72283905f) return __builtin_inff();
  const float k = rintf(x * 1.44269504089f);
  float r = __builtin_fmaf(-k, 0.693145751953125f, x);
  r = __builtin_fmaf(-k, 1.428606765330187e-06f, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return ldexpf(p, (int) k);
}

__device__ inline float lane_swiglu(float g, float u, float lim, float scale) {
  const float gv = fminf(g, lim), uv = fminf(fmaxf(u, -lim), lim);
  return __fmul_rn(__fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, lane_exp(-gv))), uv), scale);
}

// part: ((d * s21) * 1/8) * isum, each product rounded (reference kernels/lane.h:63)
__device__ inline float lane_part(float d, int s21, int isum) {
  return __fmul_rn(__fmul_rn(__fmul_rn(d, (float) s21), 0.125f), (float) isum);
}

}  // namespace osm
