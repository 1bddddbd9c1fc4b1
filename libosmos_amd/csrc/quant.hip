// libosmos MI355X - the weights' exact decode to fp32 (include/osmos/gpu/quant.h): quant_known, quant_dequant.
// contract: reference include/osmos/gpu/quant.h:23-36 - each value decode.h's (the reference's kernels/quant.h bits).
// a thread a chunk of 8 values, two float4 stores.
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
