// libosmos MI355X - one routed MoE layer over the lane's int8 contract (include/osmos_mi355x.h: osmos_lane_layer,
// osmos_lane_workspace): one persistent launch (fused.h layer_kernel) when gate/up and down share a quant type, else
// two fused launches - gate/up with the activation, then down with the tokens' ordered expert sums - in the order of the reference's src/run/hip_lane.c:115-222 and src/cpu/lane.c:98-118, so every
// output is the reference CPU lane's bits. no host round trip, no allocation: capturable in a HIP graph.
#include <algorithm>

#include "fused.h"

extern "C" {
#include "../../include/osmos_mi355x.h"
}

namespace osm {
namespace layer {

using fused::DnArgs;
using fused::GuArgs;

template <uint32_t T, int NT, int L>
bool gu_launch(const GuArgs& a, hipStream_t s) {
  const uint32_t n = a.n_tok * a.k;
  const fused::GuLds l = fused::gu_lds((uint32_t) row_bytes<T>(a.dim), a.dim, NT, fused::grid_bytes<T>(), n);
  if (l.total > 160 * 1024) return false;
  auto k = fused::gu_kernel<T, NT, L>;
  if (l.total > 64 * 1024 &&
      hipFuncSetAttribute((const void*) k, hipFuncAttributeMaxDynamicSharedMemorySize, (int) l.total) != hipSuccess)
    return false;
  k<<<dim3(a.ff / fused::kGuRows, n), fused::kThreads, l.total, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T, int L>
bool dn_launch(const DnArgs& a, hipStream_t s) {
  const fused::DnLds l = fused::dn_lds((uint32_t) row_bytes<T>(a.ff), a.ff, a.k, fused::grid_bytes<T>());
  if (l.total > 160 * 1024) return false;
  auto k = fused::dn_kernel<T, L>;
  if (l.total > 64 * 1024 &&
      hipFuncSetAttribute((const void*) k, hipFuncAttributeMaxDynamicSharedMemorySize, (int) l.total) != hipSuccess)
    return false;
  k<<<dim3(a.dim / fused::kDnRows, a.n_tok), fused::kThreads, l.total, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool gu_by(const GuArgs& a, hipStream_t s) {
  if (a.dim % Block<T>::values) return false;
  const bool wide = a.dim >= 4096;  // the contract's 32 lanes a row
  if (a.n_tok == 1) return wide ? gu_launch<T, 1, 32>(a, s) : gu_launch<T, 1, 16>(a, s);
  return wide ? gu_launch<T, 2, 32>(a, s) : gu_launch<T, 2, 16>(a, s);
}

template <uint32_t T>
bool dn_by(const DnArgs& a, hipStream_t s) {
  if (a.ff % Block<T>::values) return false;
  return a.ff >= 4096 ? dn_launch<T, 32>(a, s) : dn_launch<T, 16>(a, s);
}

// the single launch (fused::layer_kernel) over one quant type: a workgroup a tile; refused (false, nothing queued)
// unless the down tiles stay under half the workgroups the chip holds at once
int cu_count() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus[dev];
}

template <uint32_t T, int NT>
bool pk_launch(const GuArgs& ga, const DnArgs& da, fused::Ctrl* ctrl, hipStream_t s) {
  const uint32_t n = ga.n_tok * ga.k;
  const uint32_t lds = std::max(
      fused::gu_lds((uint32_t) row_bytes<T>(ga.dim), ga.dim, NT, fused::grid_bytes<T>(), n).total,
      fused::dn_lds((uint32_t) row_bytes<T>(da.ff), da.ff, da.k, fused::grid_bytes<T>()).total);
  if (lds > 160 * 1024 - 64) return false;  // (the kernel's own word besides)
  auto k = fused::layer_kernel<T, NT>;
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute((const void*) k, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds) != hipSuccess)
    return false;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, fused::kThreads, lds) != hipSuccess) return false;
  const uint32_t dn_tiles = da.n_tok * (da.dim / fused::kDnRows);
  if (2 * (uint64_t) dn_tiles > (uint64_t) per_cu * cu_count()) return false;
  const uint32_t grid = n * (ga.ff / fused::kGuRows) + dn_tiles;
  k<<<grid, fused::kThreads, lds, s>>>(ga, da, ctrl, ga.dim >= 4096 ? 32 : 16, da.ff >= 4096 ? 32 : 16);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool pk_by(const GuArgs& ga, const DnArgs& da, fused::Ctrl* ctrl, hipStream_t s) {
  if (ga.dim % Block<T>::values || da.ff % Block<T>::values) return false;
  return ga.n_tok == 1 ? pk_launch<T, 1>(ga, da, ctrl, s) : pk_launch<T, 2>(ga, da, ctrl, s);
}

#define OSM_LANE_TYPES(X) X(kIQ2_XXS) X(kIQ2_XS) X(kIQ1_M) X(kIQ1_S) X(kIQ2_S) X(kIQ3_XXS) X(kQ2_K) X(kQ4_0) X(kQ4_K) X(kQ3_K)

bool gu(uint32_t type, const GuArgs& a, hipStream_t s) {
  switch (type) {
#define X(t) \
  case t: return gu_by<t>(a, s);
    OSM_LANE_TYPES(X)
#undef X
    default: return false;
  }
}

bool dn(uint32_t type, const DnArgs& a, hipStream_t s) {
  switch (type) {
#define X(t) \
  case t: return dn_by<t>(a, s);
    OSM_LANE_TYPES(X)
#undef X
    default: return false;
  }
}

bool pk(uint32_t type, const GuArgs& ga, const DnArgs& da, fused::Ctrl* ctrl, hipStream_t s) {
  switch (type) {
#define X(t) \
  case t: return pk_by<t>(ga, da, ctrl, s);
    OSM_LANE_TYPES(X)
#undef X
    default: return false;
  }
}

// the workspace: h (a row of ff floats a pick), then the persistent launch's control words
uint64_t h_bytes(const OsmosLaneLayer* L, uint32_t n_tok) { return ((uint64_t) n_tok * L->k * L->ff * 4 + 255) / 256 * 256; }
uint64_t ctrl_bytes(const OsmosLaneLayer* L, uint32_t n_tok) {
  return (sizeof(fused::Ctrl) + fused::ctrl_lines(n_tok * L->k, n_tok) * fused::kCtrlStride * 4 + 255) / 256 * 256;
}

}  // namespace layer
}  // namespace osm

using namespace osm;

extern "C" OSM_API uint64_t osmos_lane_workspace(const OsmosLaneLayer* L, uint32_t n_tok) {
  if (!L || !n_tok || !L->k) return 0;
  return layer::h_bytes(L, n_tok) + layer::ctrl_bytes(L, n_tok);
}

extern "C" OSM_API bool osmos_lane_layer(const OsmosLaneLayer* L, const float* x, uint32_t n_tok, const int32_t* ids,
                                         const float* w, const float* add, float* out, void* workspace,
                                         uint64_t workspace_bytes, void* stream) {
  if (!L || !x || !n_tok || !ids || !w || !add || !out || !workspace || !L->k || !L->dim || !L->ff || !L->n_exp ||
      !L->gate || !L->up || !L->down || n_tok > fused::kMaxTok || L->k > fused::kMaxK || L->dim % 32 ||
      L->ff % fused::kGuRows || L->ff % 32 || L->dim % fused::kDnRows || (uintptr_t) workspace % 16 ||
      ((uintptr_t) L->gate | (uintptr_t) L->up | (uintptr_t) L->down | L->gate_bytes | L->up_bytes | L->down_bytes) % 16)
    return false;
  if (workspace_bytes < osmos_lane_workspace(L, n_tok)) return false;
  float* h = (float*) workspace;
  const hipStream_t s = (hipStream_t) stream;
  const fused::GuArgs ga = {x, ids, w, n_tok, L->k, L->dim, L->ff, (const uint8_t*) L->gate, (const uint8_t*) L->up,
                            L->gate_bytes, L->up_bytes, L->lim, h};
  const fused::DnArgs da = {h, ids, n_tok, L->k, L->dim, L->ff, (const uint8_t*) L->down, L->down_bytes, add, out};
  if (L->type_gu == L->type_down &&  // one launch where it fits, else two
      layer::pk(L->type_gu, ga, da, (fused::Ctrl*) ((uint8_t*) workspace + layer::h_bytes(L, n_tok)), s))
    return true;
  return layer::gu(L->type_gu, ga, s) && layer::dn(L->type_down, da, s);
}
