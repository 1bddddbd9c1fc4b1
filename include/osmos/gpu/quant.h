/* libosmos MI355X: the weights' exact decode (drop-in for the reference's include/osmos/gpu/quant.h:7-8).
   contract: reference include/osmos/gpu/quant.h:23-36 - each value kernels/quant.h's bits. */
#ifndef QUANT_H
#define QUANT_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces reference include/osmos/gpu/quant.h:7 (kernels/quant.hip) */
bool quant_known(uint32_t type);
/* replaces reference include/osmos/gpu/quant.h:8 (kernels/quant.hip) */
bool quant_dequant(uint32_t type, const void *src, uint64_t values, float *dst, void *stream);

#ifdef __cplusplus
}
#endif

#endif
