/* libosmos MI355X: the lane's int8 expert products (drop-in for the reference's include/osmos/gpu/q8.h:7-13).
   contract: reference include/osmos/gpu/q8.h:17-44 and kernels/lane.h:43-75 - bit for bit, on gfx950 wave64.
   types: the reference's IQ2_XXS, IQ2_XS, IQ1_M, IQ1_S, IQ2_S, IQ3_XXS, Q2_K, and (this build's extension, the same
   contract's float steps over their own codes) Q4_0, Q4_K, Q3_K. every call queued on `stream` (a hipStream_t; NULL
   the default), never waited for; false = refused, nothing queued. */
#ifndef Q8_H
#define Q8_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/q8.h:7 (kernels/q8.hip:81-88) */
bool q8_round(const float *x, uint32_t rows, uint32_t cols, uint32_t xs, int8_t *q, float *d, void *stream);
/* replaces reference include/osmos/gpu/q8.h:8-10 (kernels/q8.hip:90-107) */
bool q8_group_tok(uint32_t type, const void *const *w, const int32_t *cnt, const int32_t *xrow, const int32_t *xin,
                  uint32_t n, uint32_t max_cnt, uint32_t rows, uint32_t cols, const int8_t *q, const float *d, float *y,
                  uint32_t ys, void *stream);
/* replaces reference include/osmos/gpu/q8.h:11-13 (kernels/q8.hip:109-129) */
bool q8_gate_up(uint32_t type, const void *const *wg, const void *const *wu, const int32_t *cnt, const int32_t *xrow,
                const int32_t *xin, const int32_t *win, uint32_t n, uint32_t max_cnt, uint32_t rows, uint32_t cols,
                const int8_t *q, const float *d, const float *scale, float lim, float *h, uint32_t hs, void *stream);

#ifdef __cplusplus
}
#endif

#endif
