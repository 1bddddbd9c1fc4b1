// libosmos MI355X - the weights' exact decode (include/osmos/gpu/quant.h): quant_known, quant_dequant,
// quant_dequant_f16, quant_repack_q5k. contract: reference include/osmos/gpu/quant.h:23-47 - each value decode.h's
// (the reference's kernels/quant.h bits). a thread a chunk of 8 values: two float4 stores, or one of 8 f16s.
#include "decode.h"

extern "C" {
#include "../../include/osmos/gpu/quant.h"
}

namespace osm {
namespace qd {

__constant__ DecodeTables kDec = make_decode_tables();
constexpr int kThreads = 256;

template <uint32_t T>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t* __restrict__ src, uint64_t chunks,
                                                           float* __restrict__ dst) {
  const uint64_t c = (uint64_t) blockIdx.x * kThreads + threadIdx.x;
  if (c >= chunks) return;
  constexpr uint32_t per = Block<T>::values / kChunk;
  float v[kChunk];
  decode<T>(kDec, src + (c / per) * Block<T>::bytes, (int) (c % per), v);
  float4* o = (float4*) (dst + c * kChunk);
  o[0] = float4{v[0], v[1], v[2], v[3]}, o[1] = float4{v[4], v[5], v[6], v[7]};
}

// the same chunk rounded to f16, nearest with ties to even (each value decode's, then the conversion: the f16 that mm's
// MFMA operands hold)
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void dequant_f16_kernel(const uint8_t* __restrict__ src, uint64_t chunks,
                                                               _Float16* __restrict__ dst) {
  const uint64_t c = (uint64_t) blockIdx.x * kThreads + threadIdx.x;
  if (c >= chunks) return;
  constexpr uint32_t per = Block<T>::values / kChunk;
  float v[kChunk];
  decode<T>(kDec, src + (c / per) * Block<T>::bytes, (int) (c % per), v);
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  half8 h;
#pragma unroll
  for (int i = 0; i < kChunk; i++) h[i] = (_Float16) v[i];
  *(half8*) (dst + c * kChunk) = h;
}

// Q5_K to Q5_KR (decode.h's Layout<kQ5_KR>): a workgroup a tile's block (16 rows' block b), thread (g, r) = (tid / 16,
// tid % 16) the row's 32-value group g - its scale and minimum unpacked to two bytes, and its two slots' low nibbles
// and fifth bits gathered from Q5_K's planes; the thread of group 0 also copies the row's d and dmin. bytes moved,
// none computed
constexpr int kRepackThreads = 128;
__global__ __launch_bounds__(kRepackThreads) void repack_q5k_kernel(const uint8_t* __restrict__ src, uint64_t pieces,
                                                                    uint32_t nb, uint8_t* __restrict__ dst) {
  using L = Layout<kQ5_KR>;
  const int r = (int) threadIdx.x % 16, g = (int) threadIdx.x / 16;
  for (uint64_t p = blockIdx.x; p < pieces; p += gridDim.x) {  // piece p: tile p / nb's block p % nb
    const uint64_t t = p / nb, b = p % nb;
    const uint8_t* blk = src + ((t * 16 + r) * nb + b) * Block<kQ5_K>::bytes;
    uint8_t* out = dst + p * 16 * Block<kQ5_KR>::bytes;
    if (g == 0)
      for (int j = 0; j < 4; j++) out[4 * r + j] = blk[j];
    uint32_t sc, mn;
    group_scale_min(blk + 4, g, sc, mn);
    uint8_t* seg = out + L::kHead + g * L::kSeg;
    seg[L::kScales + 2 * r] = (uint8_t) sc, seg[L::kScales + 2 * r + 1] = (uint8_t) mn;
    const uint8_t *hi = blk + 16, *lo = blk + 48 + 32 * (g / 2);
    for (int h = 0; h < 2; h++) {
      uint64_t nib = 0;
      uint32_t fifth = 0;
      for (int v = 0; v < 16; v++) {  // slot value v: the group's chunk 2 (v / 8) + h, its value v % 8
        const int i = 8 * (2 * (v / 8) + h) + v % 8;
        nib |= (uint64_t) ((lo[i] >> (4 * (g % 2))) & 15u) << (4 * v);
        fifth |= (uint32_t) ((hi[i] >> g) & 1u) << v;
      }
      const int slot = 16 * h + r;
      for (int j = 0; j < 8; j++) seg[8 * slot + j] = (uint8_t) (nib >> (8 * j));
      seg[L::kHighs + 2 * slot] = (uint8_t) fifth, seg[L::kHighs + 2 * slot + 1] = (uint8_t) (fifth >> 8);
    }
  }
}

template <uint32_t T>
bool run_f16(const void* src, uint64_t values, void* dst, hipStream_t s) {
  if (!src || !dst || !values || values % Block<T>::values || values % kChunk) return false;
  const uint64_t chunks = values / kChunk;
  dequant_f16_kernel<T><<<(unsigned) ((chunks + kThreads - 1) / kThreads), kThreads, 0, s>>>((const uint8_t*) src,
                                                                                             chunks, (_Float16*) dst);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool run(const void* src, uint64_t values, float* dst, hipStream_t s) {
  if (!src || !dst || !values || values % Block<T>::values || values % kChunk) return false;
  const uint64_t chunks = values / kChunk;
  dequant_kernel<T><<<(unsigned) ((chunks + kThreads - 1) / kThreads), kThreads, 0, s>>>((const uint8_t*) src, chunks,
                                                                                         dst);
  return hipGetLastError() == hipSuccess;
}

#define OSM_QD_TYPES(X) \
  X(kBF16) X(kQ8_0) X(kQ4_0) X(kIQ4_NL) X(kQ2_K) X(kQ3_K) X(kQ4_K) X(kQ5_K) X(kQ6_K) X(kIQ2_XXS) X(kIQ2_XS) X(kIQ2_S) \
  X(kIQ3_XXS) X(kIQ1_S) X(kIQ1_M) X(kIQ4_XS)

}  // namespace qd
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool quant_known(uint32_t type) {
  switch (type) {
#define X(t) case t:
    OSM_QD_TYPES(X)
#undef X
    return true;
    default: return false;
  }
}

extern "C" OSM_API bool quant_dequant(uint32_t type, const void* src, uint64_t values, float* dst, void* stream) {
  const hipStream_t s = (hipStream_t) stream;
  switch (type) {
#define X(t) \
  case t: return qd::run<t>(src, values, dst, s);
    OSM_QD_TYPES(X)
#undef X
    default: return false;
  }
}

extern "C" OSM_API bool quant_dequant_f16(uint32_t type, const void* src, uint64_t values, void* dst, void* stream) {
  if ((uintptr_t) dst % 16) return false;  // (a chunk's 8 f16s one 16-byte store)
  const hipStream_t s = (hipStream_t) stream;
  switch (type) {
#define X(t) \
  case t: return qd::run_f16<t>(src, values, dst, s);
    OSM_QD_TYPES(X)
#undef X
    default: return false;
  }
}

extern "C" OSM_API bool quant_repack_q5k(const void* src, uint32_t rows, uint32_t cols, void* dst, void* stream) {
  if (!src || !dst || src == dst || !rows || rows % 16 || !cols || cols % Block<kQ5_K>::values) return false;
  const uint32_t nb = cols / Block<kQ5_K>::values;
  const uint64_t pieces = (uint64_t) (rows / 16) * nb;
  const unsigned grid = (unsigned) (pieces < 65536 ? pieces : 65536);
  qd::repack_q5k_kernel<<<grid, qd::kRepackThreads, 0, (hipStream_t) stream>>>((const uint8_t*) src, pieces, nb,
                                                                               (uint8_t*) dst);
  return hipGetLastError() == hipSuccess;
}
