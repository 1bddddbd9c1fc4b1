/* libosmos MI355X: the decode's fp32-activation matrix-vector products (drop-in for the reference's
   include/osmos/gpu/mv.h:7-21). contract: reference include/osmos/gpu/mv.h:31-62 and kernels/mv.h:1-70 (a row's
   chunks of 8 to 32 logical lanes in order, 8 fmaf a chunk, the xor tree) - bit for bit, on gfx950 wave64. types:
   F32, BF16, Q8_0, Q4_0, IQ4_NL, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ1_S, IQ1_M, IQ4_XS
   (GGUF ids). queued on `stream`, never waited for; false = refused, nothing queued. */
#ifndef MV_H
#define MV_H

#include <stdbool.h>
#include <stdint.h>

#define MV_MAX_TOKENS 8     /* reference include/osmos/gpu/mv.h:7 */
#define MV_MAX_GROUP 65535  /* reference include/osmos/gpu/mv.h:8 */

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/mv.h:10-11 (kernels/mv.hip:264-268) */
bool mv_run(uint32_t type, const void *w, uint32_t rows, uint32_t cols, const float *x, uint32_t n_tok, float *y,
            void *stream);
/* replaces reference include/osmos/gpu/mv.h:12-13 (kernels/mv.hip:233-262) */
bool mv_group(uint32_t type, const void *const *w, uint32_t n, uint32_t rows, uint32_t cols, const float *x,
              uint32_t x_mat, uint32_t x_div, float *y, void *stream);
/* replaces reference include/osmos/gpu/mv.h:14-16 (kernels/mv.hip:203-231) */
bool mv_group_tok(uint32_t type, const void *const *w, const int32_t *cnt, const int32_t *xrow, uint32_t n,
                  uint32_t max_cnt, uint32_t rows, uint32_t cols, const float *x, uint32_t xs, float *y, uint32_t ys,
                  void *stream);
/* replaces reference include/osmos/gpu/mv.h:17-18 (kernels/mv.hip:270-299) */
bool mv_strided(uint32_t type, const void *w, uint32_t rows, uint32_t cols, const float *x, uint32_t x_stride,
                uint32_t n_tok, float *y, uint32_t y_stride, void *stream);

#ifdef __cplusplus
}
#endif

#endif
