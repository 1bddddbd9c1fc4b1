// libosmos MI355X - calibration kernels for the roofline's ceilings on the box itself (not part of the product
// library: built into libosmos_amd/libosmos_calib.so, run by bench.py --ceilings):
//   calib_read: a best-shaped streaming read - every thread a run of 16-byte loads, all in flight at once (unrolled),
//     folded into one word a workgroup so nothing is dead - over `bytes` from `src`: the HBM floor of a launch that
//     reads that much, for any workgroup size;
//   calib_gather: the same read over n regions picked through a device array of region indices (the routed layer's
//     pattern: each expert's matrix one contiguous region, the expert ids read before the weights);
//   calib_mfma: chains of gfx950 dense MFMAs (int8 16x16x64 / 32x32x32, f16 16x16x32 / 32x32x16), several
//     independent accumulators a wave so the unit never waits on a result: the matrix cores' measured peak.
#include <hip/hip_runtime.h>

#include <cstdint>

#define CALIB_API extern "C" __attribute__((visibility("default")))

namespace calib {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int TH, int U>
__global__ __launch_bounds__(TH) void read_kernel(const u32x4* __restrict__ src, uint64_t words, uint32_t* out) {
  const uint64_t per_wg = (uint64_t) TH * U;
  uint32_t acc = 0;
  for (uint64_t base = (uint64_t) blockIdx.x * per_wg; base < words; base += (uint64_t) gridDim.x * per_wg) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint64_t i = base + (uint64_t) u * TH + threadIdx.x;
      r[u] = i < words ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
  }
  if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;  // (practically never: keeps the loads live)
}

// workgroup (x, y): region ids[y] (region_bytes apart from base), its words x TH U .. of (TH U a workgroup)
template <int TH, int U>
__global__ __launch_bounds__(TH) void gather_kernel(const uint8_t* __restrict__ base, const int32_t* __restrict__ ids,
                                                    uint64_t region_bytes, uint32_t* out) {
  const u32x4* src = (const u32x4*) (base + (uint64_t) (uint32_t) ids[blockIdx.y] * region_bytes);
  const uint64_t words = region_bytes / 16, b = (uint64_t) blockIdx.x * TH * U;
  uint32_t acc = 0;
  u32x4 r[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint64_t i = b + (uint64_t) u * TH + threadIdx.x;
    r[u] = i < words ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int u = 0; u < U; u++) acc ^= r[u].x ^ r[u].y ^ r[u].z ^ r[u].w;
  if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;  // (practically never: keeps the loads live)
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kChains = 4;

// kind 0: int8 16x16x64, 1: int8 32x32x32, 2: f16 16x16x32, 3: f16 32x32x16
template <int K>
__global__ __launch_bounds__(256) void mfma_kernel(uint32_t iters, int seed, int* out) {
  const int l = threadIdx.x + seed;
  if constexpr (K == 0 || K == 1) {
    const i32x4 a = {l, l + 1, l ^ 5, l ^ 9};
    const i32x4 b = {l * 3, l * 5, l + 11, l + 17};
    if constexpr (K == 0) {
      i32x4 c[kChains] = {};
      for (uint32_t i = 0; i < iters; i++)
#pragma unroll
        for (int j = 0; j < kChains; j++) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c[j], 0, 0, 0);
      int s = 0;
#pragma unroll
      for (int j = 0; j < kChains; j++) s += c[j][0] + c[j][3];
      if (s == 0x7F00F00F) out[blockIdx.x] = s;
    } else {
      i32x16 c[kChains] = {};
      for (uint32_t i = 0; i < iters; i++)
#pragma unroll
        for (int j = 0; j < kChains; j++) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[j], 0, 0, 0);
      int s = 0;
#pragma unroll
      for (int j = 0; j < kChains; j++) s += c[j][0] + c[j][15];
      if (s == 0x7F00F00F) out[blockIdx.x] = s;
    }
  } else {
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = (_Float16) (0.001f * (l + i)), b[i] = (_Float16) (0.002f * (l - i));
    if constexpr (K == 2) {
      f32x4 c[kChains] = {};
      for (uint32_t i = 0; i < iters; i++)
#pragma unroll
        for (int j = 0; j < kChains; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
      float s = 0;
#pragma unroll
      for (int j = 0; j < kChains; j++) s += c[j][0] + c[j][3];
      if (s == 1234.5f) out[blockIdx.x] = 1;
    } else {
      f32x16 c[kChains] = {};
      for (uint32_t i = 0; i < iters; i++)
#pragma unroll
        for (int j = 0; j < kChains; j++) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
      float s = 0;
#pragma unroll
      for (int j = 0; j < kChains; j++) s += c[j][0] + c[j][15];
      if (s == 1234.5f) out[blockIdx.x] = 1;
    }
  }
}

}  // namespace calib

// threads 256 or 1024, unroll 4 / 8 / 16; grid workgroups; 16-byte aligned src, bytes a multiple of 16
CALIB_API bool calib_read(const void* src, uint64_t bytes, uint32_t grid, uint32_t threads, uint32_t unroll,
                          uint32_t* out, void* stream) {
  if (!src || !out || bytes % 16 || (uintptr_t) src % 16 || !grid) return false;
  const hipStream_t s = (hipStream_t) stream;
  const calib::u32x4* p = (const calib::u32x4*) src;
  const uint64_t w = bytes / 16;
#define CALIB_R(TH, U) \
  if (threads == TH && unroll == U) { calib::read_kernel<TH, U><<<grid, TH, 0, s>>>(p, w, out); return hipGetLastError() == hipSuccess; }
  CALIB_R(256, 4) CALIB_R(256, 8) CALIB_R(256, 16) CALIB_R(512, 4) CALIB_R(512, 8) CALIB_R(1024, 4) CALIB_R(1024, 8)
#undef CALIB_R
  return false;
}

CALIB_API bool calib_gather(const void* base, const int32_t* ids, uint32_t n, uint64_t region_bytes, uint32_t threads,
                            uint32_t unroll, uint32_t* out, void* stream) {
  if (!base || !ids || !n || !out || region_bytes % 16 || (uintptr_t) base % 16) return false;
  const hipStream_t s = (hipStream_t) stream;
  const uint8_t* p = (const uint8_t*) base;
#define CALIB_G(TH, U)                                                                                      \
  if (threads == TH && unroll == U) {                                                                       \
    const dim3 grid((unsigned) ((region_bytes / 16 + TH * U - 1) / (TH * U)), n);                           \
    calib::gather_kernel<TH, U><<<grid, TH, 0, s>>>(p, ids, region_bytes, out);                           \
    return hipGetLastError() == hipSuccess;                                                                 \
  }
  CALIB_G(64, 4) CALIB_G(128, 4) CALIB_G(256, 1) CALIB_G(256, 2) CALIB_G(256, 4) CALIB_G(256, 8) CALIB_G(512, 4)
#undef CALIB_G
  return false;
}

// ops a call: blocks x 4 waves x iters x kChains x (2 M N K)
CALIB_API bool calib_mfma(uint32_t kind, uint32_t blocks, uint32_t iters, int* out, void* stream) {
  const hipStream_t s = (hipStream_t) stream;
  switch (kind) {
    case 0: calib::mfma_kernel<0><<<blocks, 256, 0, s>>>(iters, 1, out); break;
    case 1: calib::mfma_kernel<1><<<blocks, 256, 0, s>>>(iters, 1, out); break;
    case 2: calib::mfma_kernel<2><<<blocks, 256, 0, s>>>(iters, 1, out); break;
    case 3: calib::mfma_kernel<3><<<blocks, 256, 0, s>>>(iters, 1, out); break;
    default: return false;
  }
  return hipGetLastError() == hipSuccess;
}
