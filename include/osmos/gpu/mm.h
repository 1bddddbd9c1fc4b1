/* libosmos MI355X: the quantized weights' f16 matrix products (drop-in for the reference's include/osmos/gpu/mm.h:7-40 -
   the entry points the prefill and expert batches bind: mm_known, mm_fits, mm_col_tiles, mm_x16, mm_x16_rows, mm_run,
   mm_group). contract (reference include/osmos/gpu/mm.h:119-200): each weight's exact value (decode.h, the mv
   contract's values) rounded to f16, times the f16 activations (x16, tiled as mm_x16 lays them), accumulated in F32
   on gfx950's MFMA (v_mfma_f32_16x16x32_f16) in the reference's K split (kernels/mm.hip:24-73): per type and width
   SL-value slabs over W partitions, partition p the slabs p, p + W, ... as one chain of 32-value steps from zero, the
   partitions' sums then added in order - a token's sums its own, so the same bits at any batch and any tiling;
   within (cols/16 + 20) u sum |w16 x16| of the double sum over the values it reads (the reference's own bound,
   tests/gpu/test_mm_gpu.hip:321-341). types: Q8_0, Q4_0, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K,
   IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_S, IQ1_M, IQ4_XS (GGUF ids). queued on `stream`, never waited for; false =
   refused, nothing queued. */
#ifndef MM_H
#define MM_H

#include <stdbool.h>
#include <stdint.h>

#define MM_TILE 16          /* reference include/osmos/gpu/mm.h:7 */
#define MM_MAX_TOKENS 2048  /* reference include/osmos/gpu/mm.h:8 */
#define MM_MAX_GROUP 65535  /* reference include/osmos/gpu/mm.h:9 */

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/mm.h:11 (kernels/mm.hip): whether `type` has an mm kernel here */
bool mm_known(uint32_t type);
/* replaces reference include/osmos/gpu/mm.h:12: rows whole tiles (16), cols whole blocks of the type and whole slabs
   of the type's shape for that width (under 2048 columns Q6_K's 64; a width Q8_0's 128 does not divide: 64) */
bool mm_fits(uint32_t type, uint32_t rows, uint32_t cols);
/* replaces reference include/osmos/gpu/mm.h:13: the token tiles (of 16) a decoded weight step feeds at n tokens, 1 .. 8;
   0 for a type without a kernel */
uint32_t mm_col_tiles(uint32_t type, uint32_t n);
/* replaces reference include/osmos/gpu/mm.h:14: n rows of cols F32 (row t at x + t xs) to f16 (nearest) in x16's
   tiles - token t's column c at (t/16) 16 cols + (c/16) 256 + (t%16) 16 + c%16 halves - the rows past n up to a whole
   tile zero; a value past f16's range sets *overflow (device memory, left as it is otherwise). n 1 .. MM_MAX_TOKENS,
   cols a multiple of 16, xs at least cols */
bool mm_x16(const float *x, uint32_t xs, uint32_t n, uint32_t cols, void *x16, int32_t *overflow, void *stream);
/* replaces reference include/osmos/gpu/mm.h:17-18: y[t ys + r] = sum over c of W[r][c] x16[t][c], t < n (the tiles
   of x16 cols wide) */
bool mm_run(uint32_t type, const void *w, uint32_t rows, uint32_t cols, const void *x16, uint32_t n, float *y,
            uint32_t ys, void *stream);
/* replaces reference include/osmos/gpu/mm.h:34-35: slot s of x16 (slots rows, tiled, cols wide) is row idx[s] of x
   (row r at x + r xs; -1: zero), *overflow as mm_x16. false for no slots, cols not a multiple of 16, xs under cols or
   not a multiple of 4, or x not 16-byte aligned */
bool mm_x16_rows(const float *x, uint32_t xs, const int32_t *idx, uint32_t slots, uint32_t cols, void *x16,
                 int32_t *overflow, void *stream);
/* replaces reference include/osmos/gpu/mm.h:38-40: n_mat matrices of one type and shape: matrix m (w[m]) over the
   tiled x16 from x16 + xoff[m] halves (rows xts long, its first token at a tile start), its first cnt[m] tokens
   (at most max_cnt <= MM_MAX_TOKENS) into y + yoff[m] + t ys - each tile the sums mm_run gives (the type's tuned
   shape at every width: Q6_K under 2048 columns splits K otherwise than mm_run, as the reference's does). cols whole
   128-value slabs. w, cnt, xoff, yoff on the device */
bool mm_group(uint32_t type, const void *const *w, const int32_t *cnt, uint32_t n_mat, uint32_t max_cnt, uint32_t rows,
              uint32_t cols, const void *x16, const uint32_t *xoff, uint32_t xts, float *y, const uint32_t *yoff,
              uint32_t ys, void *stream);

#ifdef __cplusplus
}
#endif

#endif
