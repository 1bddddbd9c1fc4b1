/* libosmos MI355X: the element-wise ops the lane's expert path calls between its products (drop-in for those entries
   of the reference's include/osmos/gpu/ops.h:111-117, 123-124; the header's other ops are outside this library).
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

/* replaces reference include/osmos/gpu/ops.h:123 (kernels/ops.hip:878-882): the stream held until *flag - host
   memory the GPU maps (hipHostMalloc's) - holds value, with or without its top bit (the host's mark of a failed job);
   a system-scope acquire, so what the host wrote before the flag the kernels after see. the lane's hand-off of
   CPU-computed experts (reference src/run/hip_lane.c:218-219). unlike the reference's, the wait is bounded: past
   osmos_wait_limit (ten minutes unless set) it ends, and the ops_copy_rows queued after it on the same stream write NaN
   rows instead of copying, until a later wait on that stream ends with its value. the outcome is per (device, stream):
   waits and copies on other streams do not see it. false for a value with its top bit set (no post can match it: the
   reference would wait for ever), and once 1023 distinct streams of a device have waited. */
bool ops_wait(const uint32_t *flag, uint32_t value, void *stream);
/* replaces reference include/osmos/gpu/ops.h:124 (kernels/ops.hip:884-889): rows idx[0 .. n) of src to the same rows
   of dst, len floats a row (src may be host memory the GPU maps); NaN rows while the last ops_wait on this stream is
   one that expired */
bool ops_copy_rows(float *dst, const float *src, const int32_t *idx, uint32_t n, uint32_t len, void *stream);

#ifdef __cplusplus
}
#endif

#endif
