// libosmos MI355X - one routed MoE layer over the lane's int8 contract (include/osmos_mi355x.h: osmos_lane_layer,
// osmos_lane_workspace): host code sequencing the library's own entry points on one stream, the order of the reference's
// src/run/hip_lane.c:115-222 (fwd_lane_experts) with its host-side tables replaced by osmos_lane_tables (device), so a
// step needs no host round trip and can be captured in a HIP graph.
#include "common.h"

extern "C" {
#include "../../include/osmos_mi355x.h"
}

namespace {

constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// the workspace's pieces, in order
struct Carve {
  uint64_t q, qd, tok, pair, cnt, xrow, wg, wu, wd, order, h, qh, qhd, ye, total;
};

Carve carve(const OsmosLaneLayer* L, uint32_t n_tok) {
  const uint64_t n = (uint64_t) n_tok * L->k;
  Carve c;
  uint64_t at = 0;
  auto take = [&](uint64_t bytes) { const uint64_t r = at; at += up(bytes); return r; };
  c.q = take((uint64_t) n_tok * L->dim), c.qd = take((uint64_t) n_tok * (L->dim / 32) * 4);
  c.tok = take(n * 4), c.pair = take(n * 4), c.cnt = take(n * 4), c.xrow = take(n * 4);
  c.wg = take(n * 8), c.wu = take(n * 8), c.wd = take(n * 8), c.order = take(n * 4);
  c.h = take(n * L->ff * 4), c.qh = take(n * L->ff), c.qhd = take(n * (L->ff / 32) * 4);
  c.ye = take(n * L->dim * 4);
  c.total = at;
  return c;
}

}  // namespace

extern "C" OSM_API uint64_t osmos_lane_workspace(const OsmosLaneLayer* L, uint32_t n_tok) {
  if (!L || !n_tok || !L->k) return 0;
  return carve(L, n_tok).total;
}

extern "C" OSM_API bool osmos_lane_layer(const OsmosLaneLayer* L, const float* x, uint32_t n_tok, const int32_t* ids,
                                         const float* w, const float* add, float* out, void* workspace,
                                         uint64_t workspace_bytes, void* stream) {
  if (!L || !x || !n_tok || !ids || !w || !add || !out || !workspace || !L->k || !L->dim || !L->ff ||
      (uintptr_t) workspace % kAlign || (uint64_t) n_tok * L->k > OSMOS_LANE_MAX_PAIRS)
    return false;
  const Carve c = carve(L, n_tok);
  if (workspace_bytes < c.total) return false;
  uint8_t* ws = (uint8_t*) workspace;
  int8_t *q = (int8_t*) (ws + c.q), *qh = (int8_t*) (ws + c.qh);
  float *qd = (float*) (ws + c.qd), *h = (float*) (ws + c.h), *qhd = (float*) (ws + c.qhd), *ye = (float*) (ws + c.ye);
  int32_t *tok = (int32_t*) (ws + c.tok), *pair = (int32_t*) (ws + c.pair), *cnt = (int32_t*) (ws + c.cnt);
  int32_t *xrow = (int32_t*) (ws + c.xrow), *order = (int32_t*) (ws + c.order);
  const void **wg = (const void**) (ws + c.wg), **wu = (const void**) (ws + c.wu), **wd = (const void**) (ws + c.wd);
  const uint32_t n = n_tok * L->k, max_cnt = n_tok < MV_MAX_TOKENS ? n_tok : MV_MAX_TOKENS;
  const void* base[3] = {L->gate, L->up, L->down};
  const uint64_t bytes[3] = {L->gate_bytes, L->up_bytes, L->down_bytes};
  return q8_round(x, n_tok, L->dim, L->dim, q, qd, stream) &&
         osmos_lane_tables(ids, n_tok, L->k, L->n_exp, base, bytes, tok, pair, cnt, xrow, wg, wu, wd, order, stream) &&
         q8_gate_up(L->type_gu, wg, wu, cnt, xrow, tok, pair, n, max_cnt, L->ff, L->dim, q, qd, w, L->lim, h, L->ff,
                    stream) &&
         q8_round(h, n, L->ff, L->ff, qh, qhd, stream) &&
         q8_group_tok(L->type_down, wd, cnt, xrow, nullptr, n, max_cnt, L->dim, L->ff, qh, qhd, ye, L->dim, stream) &&
         ops_gather_sum_add(out, ye, order, L->k, n_tok, L->dim, add, stream);
}
