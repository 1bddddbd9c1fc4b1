/* libosmos MI355X: the Qwen-style MoE plumbing around the expert products (drop-in for the routing, table,
   activation and sum entries of the reference's include/osmos/gpu/q4x_ops.h:8-16,133-162; the rest of that header -
   the model's attention, DeltaNet and drafter ops - is outside this library). contracts: reference
   include/osmos/gpu/q4x_ops.h:356-384. */
#ifndef OSMOS_GPU_Q4X_OPS_H
#define OSMOS_GPU_Q4X_OPS_H

#include <stdbool.h>
#include <stdint.h>

#define Q4X_GROUP_TENSORS 3 /* reference include/osmos/gpu/q4x_ops.h:135: gate, up, down */
#define Q4X_TILE_RUNS 4     /* reference include/osmos/gpu/q4x_ops.h:147: parts of 1, 2, 4 or 8 tiles of 16 */

/* reference include/osmos/gpu/q4x_ops.h:136-146 (field for field) */
typedef struct Q4xExpertTiles
{
  const void *base[Q4X_GROUP_TENSORS];
  uint64_t bytes[Q4X_GROUP_TENSORS];
  const void *const *tab[Q4X_GROUP_TENSORS];
  const void **ptr[Q4X_GROUP_TENSORS];
  int32_t *cnt;
  int32_t *gidx, *hidx;
  uint32_t *xg, *yg, *xd, *yd;
  int32_t *where;
  int32_t *off;
} Q4xExpertTiles;

/* reference include/osmos/gpu/q4x_ops.h:148-152 */
typedef struct Q4xExpertBounds
{
  uint32_t first[Q4X_TILE_RUNS], count[Q4X_TILE_RUNS];
  uint32_t entries, slots;
} Q4xExpertBounds;

/* reference include/osmos/gpu/q4x_ops.h:8-16 (field for field): an op's output also written as mm's f16 activations
   (mm.h's tiled x16, rows of `cols`, the op's first row at row0), the bytes mm_x16 would make of it */
typedef struct Q4xX16
{
  void *x16;
  int32_t *overflow;
  uint32_t cols;
  uint32_t row0;
} Q4xX16;

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/q4x_ops.h:133-134 (kernels/q4x_moe.hip:204-210) */
bool q4x_route(const float *logits, uint32_t n_tok, uint32_t n_exp, uint32_t k, int32_t *ids, float *w, int32_t *rows,
               void *stream);
/* replaces reference include/osmos/gpu/q4x_ops.h:154 (kernels/q4x_moe.hip:212-218) */
void q4x_expert_bounds(uint32_t n, uint32_t n_exp, Q4xExpertBounds *b);
/* replaces reference include/osmos/gpu/q4x_ops.h:155-156 (kernels/q4x_moe.hip:220-233) */
bool q4x_expert_tiles(const int32_t *ids, uint32_t n, uint32_t k, uint32_t n_exp, uint32_t dim, uint32_t ff,
                      const Q4xExpertTiles *t, void *stream);
/* replaces reference include/osmos/gpu/q4x_ops.h:157 (kernels/q4x_moe.hip:255-259): y[i] = silu(g[i]) u[i] for i < n
   (silu(x) = x / (1 + exp(-x))); with `side` (not NULL, side->x16 not NULL) each value also into side->x16 as element
   (row0 + i / cols, i % cols) of mm_x16's tiled f16 rows, *side->overflow set for a value past f16's range. y may be
   g or u (in place). the shared expert's activation (reference src/q4x/hip_layers.c:392) */
bool q4x_swiglu(const float *g, const float *u, uint64_t n, float *y, const Q4xX16 *side, void *stream);
/* replaces reference include/osmos/gpu/q4x_ops.h:158 (kernels/q4x_moe.hip:261-272): a test's - the stream held for at
   least about `us` microseconds of the GPU's constant-rate clock, nothing computed */
bool q4x_spin(uint32_t us, void *stream);
/* replaces reference include/osmos/gpu/q4x_ops.h:159-160 (kernels/q4x_moe.hip:235-253): the experts' activation
   straight into the down's f16 - slot s's column c is silu(g[r][c]) u[r][c] (silu(x) = x / (1 + exp(-x))) for its row
   r = idx[s] (-1: zero), rounded to f16 and tiled as mm_x16_rows (mm.h) lays it, *overflow set past f16's range (the
   slots past `slots` in the last tile untouched). ff a multiple of 16, x16 16-byte aligned, overflow not NULL */
bool q4x_swiglu_rows(const float *g, const float *u, uint32_t ff, const int32_t *idx, uint32_t slots, void *x16,
                     int32_t *overflow, void *stream);
/* replaces reference include/osmos/gpu/q4x_ops.h:161-162 (kernels/q4x_moe.hip:274-285) */
bool q4x_moe_sum(const float *y, const int32_t *where, const float *w, uint32_t n_tok, uint32_t k, uint32_t dim,
                 const float *shared, const float *shared_logit, float *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif
