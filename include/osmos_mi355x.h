/* libosmos MI355X - entry points of this library that have no single counterpart in the reference's kernel ABI:
   the device-side version of the lane's host table build and the whole routed layer it feeds. everything else this
   library exports is declared, signature for signature, in include/osmos/gpu/{q8,mv,mmq,quant,q4x_ops,ops}.h. */
#ifndef OSMOS_MI355X_H
#define OSMOS_MI355X_H

#include <stdbool.h>
#include <stdint.h>

#include "osmos/gpu/mmq.h"
#include "osmos/gpu/mv.h"
#include "osmos/gpu/ops.h"
#include "osmos/gpu/q4x_ops.h"
#include "osmos/gpu/q8.h"
#include "osmos/gpu/quant.h"

#define OSMOS_LANE_MAX_PAIRS 4096 /* osmos_lane_tables' most (token, expert) pairs a step */

/* the lane's tables for one step, on the device (what reference src/run/hip_lane.c:115-200 builds on the host after
   copying the picks back; here no host round trip): the step's n_tok x k picks `ids` sorted by (expert, pick) into pair
   rows r; tok[r] the pair's token, pair[r] its pick index (t k + j); entries of at most MV_MAX_TOKENS rows of one
   expert (an expert's rows split in order), entry e: cnt[e], xrow[e] (its first pair row) and its three matrices
   wg/wu/wd[e] = base[i] + expert * bytes[i]; entries past the live ones cnt 0 up to n_tok k; order[t k + j] token t's
   pair rows in ascending row (= ascending expert id), for ops_gather_sum_add. all outputs device memory of n_tok k
   entries. false, nothing queued, for n_tok k past OSMOS_LANE_MAX_PAIRS, k 0, n_exp 0, or a launch refused. */
bool osmos_lane_tables(const int32_t *ids, uint32_t n_tok, uint32_t k, uint32_t n_exp, const void *const *base,
                       const uint64_t *bytes, int32_t *tok, int32_t *pair, int32_t *cnt, int32_t *xrow,
                       const void **wg, const void **wu, const void **wd, int32_t *order, void *stream);

/* one routed MoE layer over the lane's int8 contract, on the device, as the reference's lane runs it
   (src/run/hip_lane.c:115-222 with the tables of osmos_lane_tables, src/cpu/lane.c:98-118's phases): x's n_tok rows
   rounded (q8_round), each expert's gate and up with the activation lane_swiglu(g, u, lim, w[pick]) (q8_gate_up, inputs
   by token, weights by pick), the activations rounded, down (q8_group_tok), then each token's expert rows summed in
   ascending expert id and add[t] added after (ops_gather_sum_add) into out (n_tok rows of dim). the bits of the
   reference CPU lane for every token, whatever n_tok. `gate`, `up`, `down`: each tensor's n_exp experts back to back,
   an expert `*_bytes` apart (GGUF rows: gate/up ff rows of dim, down dim rows of ff); ids / w: the router's n_tok x k
   picks and weights. workspace: device memory of osmos_lane_workspace bytes (256-aligned), the caller's; calls sharing
   a workspace must be ordered on one stream. */
typedef struct OsmosLaneLayer
{
  uint32_t type_gu, type_down; /* the lane's types (q8.h) */
  uint32_t dim, ff, n_exp, k;
  float lim;                   /* the activation's clamp (INFINITY: none) */
  const void *gate, *up, *down;
  uint64_t gate_bytes, up_bytes, down_bytes;
} OsmosLaneLayer;

uint64_t osmos_lane_workspace(const OsmosLaneLayer *layer, uint32_t n_tok);
bool osmos_lane_layer(const OsmosLaneLayer *layer, const float *x, uint32_t n_tok, const int32_t *ids, const float *w,
                      const float *add, float *out, void *workspace, uint64_t workspace_bytes, void *stream);

/* osmos_lane_layer with no workspace argument and no allocation, for callers that cannot allocate device memory (code
   under HIP graph capture, serving loops, harnesses that forbid hipMalloc); no counterpart in the reference. Its
   workspace is a static device array of OSMOS_LANE_SCRATCH_BYTES a GPU inside this library (looked up once a device on
   the first call there, held until the process ends): a layer whose osmos_lane_workspace(layer, n_tok) exceeds that is
   refused (false, nothing queued). Every call on one GPU shares that GPU's array, so calls on one GPU must be ordered
   (one stream, or synchronised): calls that overlap on one GPU race. The same bits as osmos_lane_layer. */
#define OSMOS_LANE_SCRATCH_BYTES (16u << 20)
bool osmos_lane_layer_noalloc(const OsmosLaneLayer *layer, const float *x, uint32_t n_tok, const int32_t *ids,
                              const float *w, const float *add, float *out, void *stream);

/* the lane contract at prefill scale: q8_group_tok's sums (include/osmos/gpu/q8.h; reference kernels/q8.h:178-212,
   src/cpu/q8.c:383-407) for any token count - matrix m (w[m], rows x cols of `type`) over rows xrow[m] ..
   xrow[m] + cnt[m] - 1 of the rounded activations q / d (q8_round's layout), into the same rows of y (ys apart); the
   same bits as q8_group_tok and the reference CPU lane for every row, whatever the count. no counterpart in the
   reference (its lane stops at 8 tokens a matrix; its prompts take the f16 mm): for prompt batches of the lane's types
   on the int8 matrix cores. types IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_S, IQ1_M; rows a multiple of 16, cols of 256;
   max_cnt (the largest cnt) at most OSMOS_LANE_MAX_TOKENS. w, cnt, xrow on the device; false = refused, nothing
   queued. */
#define OSMOS_LANE_MAX_TOKENS 4096
bool osmos_lane_group(uint32_t type, const void *const *w, const int32_t *cnt, const int32_t *xrow, uint32_t n_mat,
                      uint32_t max_cnt, uint32_t rows, uint32_t cols, const int8_t *q, const float *d, float *y,
                      uint32_t ys, void *stream);

/* the layer's two halves, for callers that keep h themselves (osmos_lane_layer is the one followed by the other, h in
   its workspace): gate_up writes h, n_tok k rows of ff floats (pick t k + j's activations, weight w folded in), from
   x; down rounds h and writes out = each token's k expert rows summed in ascending expert id, then add. h 16-aligned.
   These have no counterpart in the reference, whose lane runs the two halves as separate per-table launches
   (src/run/hip_lane.c:115-222). */
bool osmos_lane_gate_up(const OsmosLaneLayer *layer, const float *x, uint32_t n_tok, const int32_t *ids, const float *w,
                        float *h, void *stream);
bool osmos_lane_down(const OsmosLaneLayer *layer, const float *h, uint32_t n_tok, const int32_t *ids, const float *add,
                     float *out, void *stream);

/* ops_wait's bound (include/osmos/gpu/ops.h), in microseconds of wall clock, for the calls queued after this one; 0:
   the default, ten minutes. no counterpart in the reference, whose wait has no bound: a stream can never be held for
   good by a host that never posts, and a failure test can end a wait early on purpose */
void osmos_wait_limit(uint64_t us);

#endif
