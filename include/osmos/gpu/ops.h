/* libosmos MI355X: the element-wise ops the lane's expert path calls between its products (drop-in for those entries
   of the reference's include/osmos/gpu/ops.h:111-117; the header's other ops are outside this library).
   contracts: reference include/osmos/gpu/ops.h:311-355. */
#ifndef OSMOS_GPU_OPS_H
#define OSMOS_GPU_OPS_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/ops.h:111-112 (kernels/ops.hip:502-507, 811-816): h = lane_swiglu(g, u, lim,
   scale[row]) over n_tok rows of n */
bool ops_swiglu_lane(const float *g, const float *u, uint32_t n, float lim, const float *scale, uint32_t n_tok,
                     float *h, void *stream);
/* replaces reference include/osmos/gpu/ops.h:113 (kernels/ops.hip:509-513) */
bool ops_gather_rows(float *dst, const float *src, const int32_t *idx, uint32_t n, uint32_t len, void *stream);
/* replaces reference include/osmos/gpu/ops.h:116-117 (kernels/ops.hip:515-525, 848-853): y[t] = sum over j < m in
   order of src[idx[t m + j]], then add[t] added */
bool ops_gather_sum_add(float *y, const float *src, const int32_t *idx, uint32_t m, uint32_t n, uint32_t dim,
                        const float *add, void *stream);

#ifdef __cplusplus
}
#endif

#endif
