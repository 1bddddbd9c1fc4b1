/* libosmos MI355X: the weights' exact decode (drop-in for the reference's include/osmos/gpu/quant.h:7-19).
   contract: reference include/osmos/gpu/quant.h:23-47 - each value kernels/quant.h's bits. */
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
/* replaces reference include/osmos/gpu/quant.h:9 (kernels/quant.hip): quant_dequant's values rounded to f16 (nearest,
   ties to even), 2 bytes a value at dst (16-byte aligned) */
bool quant_dequant_f16(uint32_t type, const void *src, uint64_t values, void *dst, void *stream);
/* replaces reference include/osmos/gpu/quant.h:10 (kernels/quant.hip:52-93): a row-major Q5_K matrix into
   QUANT_Q5_KR (tiles of 16 rows: mm_run, mm_group and mv_strided give it Q5_K's bits); false, nothing queued, for
   rows not a multiple of 16, cols not of 256, or src == dst. QUANT_Q5_KR is not a quant_dequant type */
bool quant_repack_q5k(const void *src, uint32_t rows, uint32_t cols, void *dst, void *stream);

/* reference include/osmos/gpu/quant.h:14-19 (the same values: the types' GGUF ids and the repacked layout's size) */
#define QUANT_Q5_K 13u
#define QUANT_Q5_K_VALUES 256u
#define QUANT_Q5_K_BYTES 176u
#define QUANT_Q5_KR (0x100u | QUANT_Q5_K)
#define QUANT_Q5_KR_BYTES_A_BLOCK 180u
#define QUANT_Q5_KR_BYTES(rows, cols) ((uint64_t)(rows) * ((cols) / QUANT_Q5_K_VALUES) * QUANT_Q5_KR_BYTES_A_BLOCK)

#ifdef __cplusplus
}
#endif

#endif
