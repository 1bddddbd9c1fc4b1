/* TEST INFRASTRUCTURE ONLY - the CPU oracle: a scalar C restatement of the reference's arithmetic contracts for the
   quantized-weight matrix products, used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
   checker. nothing in the product (libosmos_amd/) links, loads or calls it.

   contracts restated (reference = mrsirg97-rgb/libosmos):
   - lane (int8 activations): kernels/lane.h:43-75, kernels/q8.h:28-277, src/cpu/q8.c:9-435,
     include/osmos/gpu/q8.h:17-44;
   - mv (fp32 activations): kernels/mv.h:1-70, kernels/quant.h:60-348, src/cpu/expert.c:10-253,
     include/osmos/gpu/mv.h:31-62;
   - mmq (Q4_K on int8 matrix cores): include/osmos/gpu/mmq.h:37-55, kernels/mmq.hip:33-151;
   - mm (the f16 matmul's K split and partition order): include/osmos/gpu/mm.h:87-200, kernels/mm.hip:24-73,
     kernels/mm.h:84-90 (a step's rounding modeled: exact where no step drops a bit - see mm.c);
   - the lane's layer (round x, gate/up + swiglu, round h, down, token sums by ascending expert): src/cpu/lane.c:71-118,
     src/run/hip_lane.c:164-220, kernels/ops.hip:502-516;
   - MoE plumbing: kernels/q4x_moe.hip:38-200 (route, expert tables, weighted sum).
   build-defined (no reference contract; "parity unpinned" beyond this restatement and its closed-form checks):
   - Q4_0, Q4_K and Q3_K on the lane's int8 activations (oracle/lane.c, orc_lane_block).

   pinning: every function here is checked in tests/test_oracle.py against golden vectors written by the reference's
   own compiled CPU path (tests/golden/, oracle/ref.mk) or against closed forms (float64 dequantisation, brute-force
   integer dots, the contract's bound), as that file's docstrings list. */
#ifndef OSMOS_ORACLE_H
#define OSMOS_ORACLE_H

#include <stdbool.h>
#include <stdint.h>

/* GGUF type ids (reference include/osmos/model/qtype.h:28-53) */
enum
{
  ORC_F32 = 0,
  ORC_Q4_0 = 2,
  ORC_Q8_0 = 8,
  ORC_Q2_K = 10,
  ORC_Q3_K = 11,
  ORC_Q4_K = 12,
  ORC_Q5_K = 13,
  ORC_Q6_K = 14,
  ORC_IQ2_XXS = 16,
  ORC_IQ2_XS = 17,
  ORC_IQ3_XXS = 18,
  ORC_IQ1_S = 19,
  ORC_IQ4_NL = 20,
  ORC_IQ2_S = 22,
  ORC_IQ4_XS = 23,
  ORC_IQ1_M = 29,
  ORC_BF16 = 30,
};

void orc_init(void);
/* a type's block values and bytes (0 for a type the oracle does not know) */
uint32_t orc_block_values(uint32_t type);
uint32_t orc_block_bytes(uint32_t type);
float orc_f16(uint32_t bits);

/* lane contract */
float orc_lane_exp(float x);
float orc_lane_swiglu(float g, float u, float lim, float scale);
bool orc_lane_known(uint32_t type);
bool orc_q8_round(const float *x, uint32_t rows, uint32_t cols, uint32_t xs, int8_t *q, float *d);
bool orc_q8_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t *q, const float *d,
                 uint32_t n, float *y, uint32_t ys);
/* one 32-value block's contribution before x's scale (the contract's `sub`) */
float orc_lane_sub(uint32_t type, const uint8_t *row, uint32_t s, const int8_t *xb);

/* mv contract */
bool orc_mv_known(uint32_t type);
bool orc_dequant(uint32_t type, const void *src, uint64_t values, float *dst);
bool orc_mv_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const float *x, uint32_t xs,
                 uint32_t n, float *y, uint32_t ys);

/* mm (the f16 matmul's order): rows r0 .. r1 of a matrix of `type` against n tokens of x (row t at x + t xs, each
   value rounded to f16), the reference's K split for the type and width (group: mm_group's); y[t ys + r] */
float orc_f16_round(float v);
void orc_mm_shape(uint32_t type, uint32_t cols, bool group, uint32_t *sl, uint32_t *w); /* the K split: slab, parts */
bool orc_mm_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const float *x, uint32_t xs,
                 uint32_t n, bool group, float *y, uint32_t ys);

/* mmq contract (Q4_K) */
uint64_t orc_mmq_x8_at(uint32_t s, uint32_t c, uint32_t cols);
uint64_t orc_mmq_dx_at(uint32_t s, uint32_t g, uint32_t groups);
bool orc_mmq_x8_rows(const float *x, uint32_t xs, const int32_t *idx, uint32_t slots, uint32_t cols, int8_t *x8,
                     float *dx, float *sx);
/* rows r0 .. r1 of a Q4_K matrix against slot `slot`'s x8 / dx / sx: y[r] */
bool orc_mmq_rows(const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t *x8, const float *dx,
                  const float *sx, uint32_t slot, float *y);

/* the lane's layer over one expert set (src/cpu/lane.c's job): n_rows rows of x (a (token, expert) pair each);
   expert e's rows row0[e] .. row0[e] + cnt[e]; gate/up ff rows of dim, down dim rows of ff; y row r at y + r * dim */
bool orc_lane_layer(uint32_t type_gu, uint32_t type_down, uint32_t dim, uint32_t ff, float lim, const float *x,
                    const float *scale, uint32_t n_rows, const void *const *gate, const void *const *up,
                    const void *const *down, const uint32_t *row0, const uint32_t *cnt, uint32_t n_e, float *y);
/* y[t][:] = sum over j < m, in j's order, of src[idx[t m + j]][:] plus add[t][:] after (ops_gather_sum_add) */
void orc_gather_sum_add(float *y, const float *src, const int32_t *idx, uint32_t m, uint32_t n, uint32_t dim,
                        const float *add);

/* MoE plumbing */
void orc_route(const float *logits, uint32_t n_tok, uint32_t n_exp, uint32_t k, int32_t *ids, float *w);
void orc_moe_sum(const float *y, const int32_t *where, const float *w, uint32_t n_tok, uint32_t k, uint32_t dim,
                 const float *shared, const float *shared_logit, float *out);

/* threaded row split of orc_q8_rows (the CPU baseline: rows split evenly, one thread a share) */
bool orc_q8_rows_mt(uint32_t type, const void *w, uint32_t cols, uint32_t rows, const int8_t *q, const float *d,
                    uint32_t n, float *y, uint32_t ys, int threads);

#endif
