/* libosmos MI355X: the experts' matmul on the int8 matrix cores (drop-in for the reference's
   include/osmos/gpu/mmq.h:7-33). contract: reference include/osmos/gpu/mmq.h:37-55 (Q4_K; the activations int8 a
   32-group; per group v = (d sc) dx, acc = fma(v, I, acc), acc = fma(dmin m, -sx, acc); K split by 256-blocks
   p, p + 4, ...; the four partial sums in order) - bit for bit, on gfx950 MFMA (v_mfma_i32_16x16x32_i8). */
#ifndef OSMOS_GPU_MMQ_H
#define OSMOS_GPU_MMQ_H

#include <stdbool.h>
#include <stdint.h>

#define MMQ_GROUP 32     /* reference include/osmos/gpu/mmq.h:7 */
#define MMQ_MAX_TILES 4  /* reference include/osmos/gpu/mmq.h:8 */
#define MMQ_SLOTS 16     /* reference include/osmos/gpu/mmq.h:9 */

#if defined(__HIPCC__)
#define MMQ_HD __host__ __device__
#else
#define MMQ_HD
#endif
/* the layouts (reference include/osmos/gpu/mmq.h:16-26): slot s's value c in x8, its group g in dx / sx */
static inline MMQ_HD uint64_t mmq_x8_at(uint32_t s, uint32_t c, uint32_t cols)
{
  return (uint64_t)(s / MMQ_SLOTS) * MMQ_SLOTS * cols + (uint64_t)(c / MMQ_GROUP) * (MMQ_SLOTS * MMQ_GROUP) +
         (s % MMQ_SLOTS) * MMQ_GROUP + c % MMQ_GROUP;
}
static inline MMQ_HD uint64_t mmq_dx_at(uint32_t s, uint32_t g, uint32_t groups)
{
  return (uint64_t)(s / MMQ_SLOTS) * MMQ_SLOTS * groups + (uint64_t)g * MMQ_SLOTS + s % MMQ_SLOTS;
}

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/mmq.h:28-29 (kernels/mmq.hip:167-174) */
bool mmq_x8_rows(const float *x, uint32_t xs, const int32_t *idx, uint32_t slots, uint32_t cols, int8_t *x8, float *dx,
                 float *sx, void *stream);
/* replaces reference include/osmos/gpu/mmq.h:30-32 (kernels/mmq.hip:176-186) */
bool mmq_group(uint32_t type, const void *const *w, const int32_t *cnt, uint32_t n_mat, uint32_t max_cnt,
               uint32_t rows, uint32_t cols, const int8_t *x8, const float *dx, const float *sx, const uint32_t *soff,
               float *y, const uint32_t *yoff, uint32_t ys, void *stream);
/* replaces reference include/osmos/gpu/mmq.h:33 (kernels/mmq.hip:165) */
bool mmq_known(uint32_t type);

#ifdef __cplusplus
}
#endif

#endif
