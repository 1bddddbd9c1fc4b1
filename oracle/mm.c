/* TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h): the f16 matmul's order (mm_run / mm_group).

   reference: include/osmos/gpu/mm.h:87-200 (the contract: each weight's exact value rounded to f16, times the f16
   activations, F32 sums), kernels/mm.hip:24-73 (the K split a type and width take: Tuned / Short / Odd shapes),
   kernels/mm.h:84-90,255-266 (partition p its slabs p, p + W, ... as one chain from zero; the partitions then summed
   in order, s = part 0, s += part 1, ...).

   a matrix-core step (32 values here: gfx950's v_mfma_f32_16x16x32_f16) is modeled as its products' exact sum plus
   the running sum, rounded once to F32. measured on the MI355X, the unit aligns the step's terms to the largest one
   and drops their bits below 2^(E - 24) (toward zero) before that rounding, so the model is the unit's bits exactly
   wherever no step drops a bit - integer-valued weights and activations below 2^24, which the tests use to pin the
   partition order bit for bit - and within the reference's bound elsewhere.
   built with -ffp-contract=off. */
#include <math.h>
#include <stdlib.h>

#include "oracle.h"

typedef struct
{
  uint32_t sl, w;
} KSplit;

static KSplit tuned(uint32_t type)
{
  switch (type)
  {
  case ORC_Q5_K:
    return (KSplit){32, 8};
  case ORC_Q4_K:
    return (KSplit){32, 16};
  case ORC_IQ1_M:
  case ORC_IQ1_S:
  case ORC_IQ2_XXS:
  case ORC_IQ2_XS:
  case ORC_IQ2_S:
    return (KSplit){128, 4};
  case ORC_IQ4_NL:
  case ORC_IQ4_XS:
  case ORC_Q4_0:
    return (KSplit){64, 4};
  case ORC_Q2_K:
  case ORC_Q3_K:
    return (KSplit){64, 8};
  default: /* Q8_0, Q6_K, IQ3_XXS */
    return (KSplit){128, 8};
  }
}

/* mm_run's shape for a width (group: mm_group's, the tuned one at every width) */
static KSplit shape_of(uint32_t type, uint32_t cols, bool group)
{
  if (group)
    return tuned(type);
  KSplit s = cols < 2048 && type == ORC_Q6_K ? (KSplit){64, 8} : tuned(type);
  if (cols % s.sl)
    s = type == ORC_Q8_0 ? (KSplit){64, 2} : s;
  return s;
}

void orc_mm_shape(uint32_t type, uint32_t cols, bool group, uint32_t *sl, uint32_t *w)
{
  const KSplit k = shape_of(type, cols, group);
  *sl = k.sl, *w = k.w;
}

/* a float's f16 value (nearest, ties to even; past the range: infinity) */
float orc_f16_round(float v)
{
  if (v != v)
    return v;
  const double a = fabs((double)v);
  if (a >= 65520.0)
    return v < 0 ? -INFINITY : INFINITY;
  int e;
  frexp(a, &e); /* a = m 2^e, m in [0.5, 1) */
  const double ulp = e - 1 >= -14 ? ldexp(1.0, e - 1 - 10) : ldexp(1.0, -24);
  const double r = nearbyint((double)v / ulp) * ulp; /* (the default rounding: to nearest, ties to even) */
  return (float)r;
}

bool orc_mm_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const float *x, uint32_t xs,
                 uint32_t n, bool group, float *y, uint32_t ys)
{
  const uint32_t bv = orc_block_values(type), bb = orc_block_bytes(type);
  if (!w || !x || !y || !bv || cols % bv || r1 < r0)
    return false;
  const KSplit k = shape_of(type, cols, group);
  if (cols % k.sl || k.sl % 32)
    return false;
  const uint64_t rb = (uint64_t)(cols / bv) * bb;
  float *wr = malloc((size_t)cols * sizeof *wr), *xr = malloc((size_t)cols * sizeof *xr);
  if (!wr || !xr)
    return free(wr), free(xr), false;
  bool ok = true;
  const uint32_t slabs = cols / k.sl;
  for (uint32_t r = r0; ok && r < r1; r++)
  {
    ok = orc_dequant(type, (const uint8_t *)w + r * rb, cols, wr);
    for (uint32_t c = 0; c < cols; c++)
      wr[c] = orc_f16_round(wr[c]);
    for (uint32_t t = 0; ok && t < n; t++)
    {
      for (uint32_t c = 0; c < cols; c++)
        xr[c] = orc_f16_round(x[(uint64_t)t * xs + c]);
      float s = 0.0f;
      for (uint32_t p = 0; p < k.w; p++)
      {
        float acc = 0.0f;
        for (uint32_t sb = p; sb < slabs; sb += k.w)
          for (uint32_t k0 = sb * k.sl; k0 < (sb + 1) * k.sl; k0 += 32)
          {
            double e = acc;
            for (uint32_t i = 0; i < 32; i++)
              e += (double)wr[k0 + i] * (double)xr[k0 + i]; /* (exact: f16 products in a double, integer tests) */
            acc = (float)e;
          }
        s = p == 0 ? acc : s + acc;
      }
      y[(uint64_t)t * ys + r] = s;
    }
  }
  free(wr), free(xr);
  return ok;
}
