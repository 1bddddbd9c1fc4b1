// libosmos MI355X - one routed MoE layer over the lane's int8 contract (include/osmos_mi355x.h: osmos_lane_layer,
// osmos_lane_workspace): two fused launches (fused.h) - gate/up with the activation, then down with the tokens'
// ordered expert sums - in the order of the reference's src/run/hip_lane.c:115-222 and src/cpu/lane.c:98-118, so every
// output is the reference CPU lane's bits. no host round trip, no allocation: capturable in a HIP graph.
#include <mutex>

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
  k<<<dim3(a.ff / fused::GuShape<NT>::rows, n), fused::GuShape<NT>::threads, l.total, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

// the one-token gate/up: 16 lanes for dim a multiple of 512 up to 2048, 32 lanes for a multiple of 1024 from 4096 to
// 8192, the tile rows in at most kG1Slots staging slots a matrix (false: not taken, the caller uses gu_kernel)
template <uint32_t T, int L>
bool gu1_launch_l(const GuArgs& a, hipStream_t s) {
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim), words = fused::kG1Rows * rb / 16;
  const dim3 grid(a.ff / fused::kG1Rows, a.k);
  constexpr int kT = fused::kG1Threads;
  if constexpr (L == 32) {  // (x already rounded: the P kernels copy it)
    if (a.xq) {
      if (words <= (uint32_t) kT)
        fused::gu1_kernel<T, 1, L, true><<<grid, kT, 0, s>>>(a);
      else if (words <= 2u * kT)
        fused::gu1_kernel<T, 2, L, true><<<grid, kT, 0, s>>>(a);
      else
        fused::gu1_kernel<T, fused::kG1Slots, L, true><<<grid, kT, 0, s>>>(a);
      return hipGetLastError() == hipSuccess;
    }
  }
  if (words <= (uint32_t) kT)
    fused::gu1_kernel<T, 1, L><<<grid, kT, 0, s>>>(a);
  else if (words <= 2u * kT)
    fused::gu1_kernel<T, 2, L><<<grid, kT, 0, s>>>(a);
  else
    fused::gu1_kernel<T, fused::kG1Slots, L><<<grid, kT, 0, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

// the batch gate/up on gu1_kernel's tile (gub_kernel), NB tokens a pass
template <uint32_t T, int L>
bool gub_launch_l(const GuArgs& a, hipStream_t s) {
  constexpr int NB = L == 16 ? 4 : 2;
  // the workgroup's waves, a row each: 8 where the tile's fixed costs (its codebook table, its tokens' x, the routing
  // ids) over twice the rows pay - 16 lanes (Qwen layer batch 4: 34.8 -> 30.9 us), and 32 lanes with a codebook of
  // 8 KB or more (IQ1_S at DeepSeek batch 4: 160 -> 151 us); else 4 (at 32 lanes with a small codebook, 8 rows'
  // LDS costs more occupancy than it saves: IQ2_XXS 224 -> 237 us). 16 was slower everywhere it fits
  constexpr int W = L == 16 || fused::grid_bytes<T>() >= 8192 ? 8 : 4;
  constexpr int kT = kWave * W;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim), words = W * rb / 16;
  const dim3 grid(a.ff / W, a.n_tok * a.k);
  if (a.xq) {  // (x already rounded: the P kernels copy it)
    if (words <= (uint32_t) kT)
      fused::gub_kernel<T, 1, L, NB, true, W><<<grid, kT, 0, s>>>(a);
    else if (words <= 2u * kT)
      fused::gub_kernel<T, 2, L, NB, true, W><<<grid, kT, 0, s>>>(a);
    else
      fused::gub_kernel<T, fused::kG1Slots, L, NB, true, W><<<grid, kT, 0, s>>>(a);
    return hipGetLastError() == hipSuccess;
  }
  if (words <= (uint32_t) kT)
    fused::gub_kernel<T, 1, L, NB, false, W><<<grid, kT, 0, s>>>(a);
  else if (words <= 2u * kT)
    fused::gub_kernel<T, 2, L, NB, false, W><<<grid, kT, 0, s>>>(a);
  else
    fused::gub_kernel<T, fused::kG1Slots, L, NB, false, W><<<grid, kT, 0, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool gu1_launch(const GuArgs& a, hipStream_t s, bool* taken) {
  *taken = false;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim);
  if ((fused::kG1Rows * rb) % 16 || fused::kG1Rows * rb / 16 > (uint32_t) (fused::kG1Slots * fused::kG1Threads) ||
      a.ff % fused::kG1Rows)
    return true;
  if (a.dim % 512 == 0 && a.dim <= fused::G1Max<16>::dim) {
    *taken = true;
    return a.n_tok == 1 ? gu1_launch_l<T, 16>(a, s) : gub_launch_l<T, 16>(a, s);
  }
  if (a.dim % 1024 == 0 && a.dim >= 4096 && a.dim <= fused::G1Max<32>::dim) {
    *taken = true;
    return a.n_tok == 1 ? gu1_launch_l<T, 32>(a, s) : gub_launch_l<T, 32>(a, s);
  }
  return true;
}

template <uint32_t T, int L, int S>
bool dn_launch_s(const DnArgs& a, hipStream_t s, uint32_t lds) {
  auto k = a.hq ? fused::dn_kernel<T, L, S, true> : fused::dn_kernel<T, L, S>;  // (h already rounded: copied)
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute((const void*) k, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds) != hipSuccess)
    return false;
  k<<<dim3(a.dim / fused::kDnRows, a.n_tok), fused::kDnThreads, lds, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T, int L>
bool dn_launch(const DnArgs& a, hipStream_t s) {
  const uint32_t rb = (uint32_t) row_bytes<T>(a.ff);
  const fused::DnLds l = fused::dn_lds(rb, a.ff, a.k, fused::grid_bytes<T>());
  if (l.total > 160 * 1024) return false;
  const uint32_t words = a.k * fused::kDnRows * rb / 16;  // the tile's 16-byte words: slots enough for one round
  if (words <= (uint32_t) fused::kDnThreads) return dn_launch_s<T, L, 1>(a, s, l.total);
  if (words <= 2u * fused::kDnThreads) return dn_launch_s<T, L, 2>(a, s, l.total);
  return dn_launch_s<T, L, fused::kPer>(a, s, l.total);
}

template <uint32_t T>
bool gu_by(const GuArgs& a, hipStream_t s) {
  if (a.dim % Block<T>::values) return false;
  const bool wide = a.dim >= 4096;  // the contract's 32 lanes a row
  bool taken = false;
  const bool ok = gu1_launch<T>(a, s, &taken);
  if (taken) return ok;
  if (a.n_tok == 1) return wide ? gu_launch<T, 1, 32>(a, s) : gu_launch<T, 1, 16>(a, s);
  return wide ? gu_launch<T, 2, 32>(a, s) : gu_launch<T, 2, 16>(a, s);
}

template <uint32_t T>
bool dn_by(const DnArgs& a, hipStream_t s) {
  if (a.ff % Block<T>::values) return false;
  return a.ff >= 4096 ? dn_launch<T, 32>(a, s) : dn_launch<T, 16>(a, s);
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

// the workspace: h, a row of ff floats a pick; where rounding x or h once beats each workgroup rounding all of it
// (dim >= 4096 or 16 tokens and more: every gate/up tile rounds its tokens' whole rows; k ff > 8192: every down tile rounds all
// of its token's activations), their rounded codes and scales (q8_round's) after it, each part 256-aligned
uint64_t a256(uint64_t b) { return (b + 255) / 256 * 256; }
uint64_t h_bytes(const OsmosLaneLayer* L, uint32_t n_tok) { return a256((uint64_t) n_tok * L->k * L->ff * 4); }
bool round_x(const OsmosLaneLayer* L, uint32_t n_tok) { return L->dim >= 4096 || n_tok >= 16; }
bool round_h(const OsmosLaneLayer* L, uint32_t n_tok) { return L->k * L->ff > 8192 || n_tok >= 16; }
uint64_t x_part(const OsmosLaneLayer* L, uint32_t n_tok) {
  return round_x(L, n_tok) ? a256((uint64_t) n_tok * L->dim) + a256((uint64_t) n_tok * L->dim / 32 * 4) : 0;
}
uint64_t h_part(const OsmosLaneLayer* L, uint32_t n_tok) {
  const uint64_t n = (uint64_t) n_tok * L->k * L->ff;
  return round_h(L, n_tok) ? a256(n) + a256(n / 32 * 4) : 0;
}

}  // namespace layer
}  // namespace osm

using namespace osm;

extern "C" OSM_API uint64_t osmos_lane_workspace(const OsmosLaneLayer* L, uint32_t n_tok) {
  if (!L || !n_tok || !L->k) return 0;
  return layer::h_bytes(L, n_tok) + layer::x_part(L, n_tok) + layer::h_part(L, n_tok);
}

namespace {
uint32_t block_values(uint32_t type) {  // a lane type's values a block (0: not a lane type)
  switch (type) {
#define X(t) \
  case t: return Block<t>::values;
    OSM_LANE_TYPES(X)
#undef X
    default: return 0;
  }
}

// every check before anything is queued: a refused layer queues nothing (a shape only the down half refuses included)
bool layer_ok(const OsmosLaneLayer* L, uint32_t n_tok) {
  const uint32_t vg = L ? block_values(L->type_gu) : 0, vd = L ? block_values(L->type_down) : 0;
  return L && vg && vd && L->dim % vg == 0 && L->ff % vd == 0 && n_tok && L->k && L->dim && L->ff && L->n_exp &&
         L->gate && L->up && L->down && n_tok <= fused::kMaxTok &&
         L->k <= fused::kMaxK && L->dim % 32 == 0 && L->ff % fused::kGuRowsMax == 0 && L->ff % 32 == 0 &&
         L->dim % fused::kDnRows == 0 &&
         ((uintptr_t) L->gate | (uintptr_t) L->up | (uintptr_t) L->down | L->gate_bytes | L->up_bytes | L->down_bytes) %
                 16 == 0;
}
}  // namespace

extern "C" OSM_API bool osmos_lane_gate_up(const OsmosLaneLayer* L, const float* x, uint32_t n_tok, const int32_t* ids,
                                           const float* w, float* h, void* stream) {
  if (!layer_ok(L, n_tok) || !x || !ids || !w || !h || (uintptr_t) h % 16) return false;
  const fused::GuArgs ga = {x, ids, w, n_tok, L->k, L->dim, L->ff, (const uint8_t*) L->gate, (const uint8_t*) L->up,
                            L->gate_bytes, L->up_bytes, L->lim, h, nullptr, nullptr};
  return layer::gu(L->type_gu, ga, (hipStream_t) stream);
}

extern "C" OSM_API bool osmos_lane_down(const OsmosLaneLayer* L, const float* h, uint32_t n_tok, const int32_t* ids,
                                        const float* add, float* out, void* stream) {
  if (!layer_ok(L, n_tok) || !h || !ids || !add || !out || (uintptr_t) h % 16) return false;
  const fused::DnArgs da = {h, ids, n_tok, L->k, L->dim, L->ff, (const uint8_t*) L->down, L->down_bytes, add, out,
                            nullptr, nullptr};
  return layer::dn(L->type_down, da, (hipStream_t) stream);
}

extern "C" OSM_API bool osmos_lane_layer(const OsmosLaneLayer* L, const float* x, uint32_t n_tok, const int32_t* ids,
                                         const float* w, const float* add, float* out, void* workspace,
                                         uint64_t workspace_bytes, void* stream) {
  if (!layer_ok(L, n_tok) || !workspace || workspace_bytes < osmos_lane_workspace(L, n_tok)) return false;
  float* h = (float*) workspace;
  uint8_t* at = (uint8_t*) workspace + layer::h_bytes(L, n_tok);
  const hipStream_t s = (hipStream_t) stream;
  int8_t* xq = nullptr;
  float* xd = nullptr;
  if (layer::round_x(L, n_tok)) {  // x rounded once (the same bits as the kernels' own rounding: q8_round's)
    xq = (int8_t*) at, at += layer::a256((uint64_t) n_tok * L->dim);
    xd = (float*) at, at += layer::a256((uint64_t) n_tok * L->dim / 32 * 4);
    if (!q8_round(x, n_tok, L->dim, L->dim, xq, xd, stream)) return false;
  }
  const fused::GuArgs ga = {x, ids, w, n_tok, L->k, L->dim, L->ff, (const uint8_t*) L->gate, (const uint8_t*) L->up,
                            L->gate_bytes, L->up_bytes, L->lim, h, xq, xd};
  if (!layer::gu(L->type_gu, ga, s)) return false;
  int8_t* hq = nullptr;
  float* hd = nullptr;
  if (layer::round_h(L, n_tok)) {  // h rounded once, rows by pick (down's rounding: q8_round's)
    const uint64_t n = (uint64_t) n_tok * L->k * L->ff;
    hq = (int8_t*) at, at += layer::a256(n);
    hd = (float*) at;
    if (!q8_round(h, n_tok * L->k, L->ff, L->ff, hq, hd, stream)) return false;
  }
  const fused::DnArgs da = {h, ids, n_tok, L->k, L->dim, L->ff, (const uint8_t*) L->down, L->down_bytes, add, out,
                            hq, hd};
  return layer::dn(L->type_down, da, s);
}

// ---- the layer with no allocation and no caller workspace: the workspace is this file's static device array ----
namespace osm {
namespace layer {

// OSMOS_LANE_SCRATCH_BYTES of device memory, one copy a GPU, held until the process ends. Host code never uses the
// symbol's name as an address: each device's copy is looked up once (hipGetSymbolAddress, that device current) and
// that address is what the kernels get
static __device__ __align__(256) uint8_t scratch[OSMOS_LANE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices];

// the calling thread's current device's copy (nullptr: no device, or the lookup failed)
void* scratch_here() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    scratch_dev[dev] = p;
  }
  return scratch_dev[dev];
}

}  // namespace layer
}  // namespace osm

extern "C" OSM_API bool osmos_lane_layer_noalloc(const OsmosLaneLayer* L, const float* x, uint32_t n_tok,
                                                 const int32_t* ids, const float* w, const float* add, float* out,
                                                 void* stream) {
  const uint64_t need = osmos_lane_workspace(L, n_tok);  // (0 for a descriptor or count refused below)
  if (!need || need > OSMOS_LANE_SCRATCH_BYTES) return false;
  void* ws = layer::scratch_here();
  if (!ws) return false;
  return osmos_lane_layer(L, x, n_tok, ids, w, add, out, ws, need, stream);
}
