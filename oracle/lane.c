/* TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h): the lane's int8 contract, scalar.

   reference: kernels/lane.h:43-75 (rounding, parts, swiglu, lane_exp), kernels/q8.h:28-162 (each type's codes and
   block_sum), kernels/q8.h:175-277 (the lane assignment, the tree, the rounding kernel), src/cpu/q8.c:9-435 (the CPU
   twin), tests/test_cpu_q8.c:139-176 (the reference's own scalar replay, row_ref / round_ref).

   a row's sum for one token: block s (32 values) to logical lane s % L (L = 32 for cols >= 4096, else 16), in ascending
   s: acc[s % L] = fmaf(xd[s], sub_s, acc[s % L]); then for o = L/2 .. 1, acc[l] = acc[l] + acc[l ^ o]; the row's value
   acc[0]. sub_s: each 16-value half's exact integer dot isum_h of the block's codes and x's int8, then
   part_h = ((d * s21_h) * 0.125) * isum_h (Q2_K: minus the same of dmin, m8_h and x's sum), sub = part_0 + part_1.

   build-defined (parity unpinned beyond this restatement): Q4_0 (codes q - 8, one part: ((d * 8) * 0.125) * isum over
   all 32), Q4_K (codes q, one part with its minimum: 8 sc and 8 m of the 32's group), Q3_K (codes q2 - (h ? 0 : 4),
   two halves, s21_h = 8 (sc_h - 32)). built with -ffp-contract=off: every product and sum rounded on its own. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "orc_internal.h"

#define LANE_VALUES 32
#define LANE_LANES(cols) ((cols) >= 4096 ? 32 : 16)

/* reference kernels/lane.h:17-41: e^x by a ln2 split and a degree-7 Horner series, times 2^k */
float orc_lane_exp(float x)
{
  if (x > 88.72283905f)
    return INFINITY;
  const float k = rintf(x * 1.44269504089f);
  float r = fmaf(-k, 0.693145751953125f, x);
  r = fmaf(-k, 1.428606765330187e-06f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

/* reference kernels/lane.h:71-75 */
float orc_lane_swiglu(float g, float u, float lim, float scale)
{
  const float gv = fminf(g, lim), uv = fminf(fmaxf(u, -lim), lim);
  return gv / (1.0f + orc_lane_exp(-gv)) * uv * scale;
}

/* reference kernels/lane.h:63 */
static float part(float d, int s21, int isum) { return d * (float)s21 * 0.125f * (float)isum; }

bool orc_lane_known(uint32_t type)
{
  switch (type)
  {
  case ORC_IQ2_XXS:
  case ORC_IQ2_XS:
  case ORC_IQ1_M:
  case ORC_IQ1_S:
  case ORC_IQ2_S:
  case ORC_IQ3_XXS:
  case ORC_Q2_K:
  case ORC_Q4_0:
  case ORC_Q4_K:
  case ORC_Q3_K: return true;
  default: return false;
  }
}

/* a 32-value block's codes: w[i] the int8 code of value i; delta[k] chunk k's +-1 (IQ1: codes 8 grid + delta), else 0;
   s21 each half's scale integer, d the block scale; Q2_K / Q4_K: m8 and dmin; whole: one part over the 32 */
typedef struct
{
  int w[32], delta[4], s21[2], m8[2];
  float d, dmin;
  int has_min, whole;
} Codes;

static void signed8(uint64_t grid, uint32_t signs, int *w)
{
  for (int i = 0; i < 8; i++)
  {
    const int v = (int)((grid >> (8 * i)) & 0xFF);
    w[i] = (signs >> i) & 1 ? -v : v;
  }
}

static void iq1(uint64_t grid, int *w)
{
  for (int i = 0; i < 8; i++)
    w[i] = (int)(int8_t)(uint8_t)(grid >> (8 * i));
}

/* block j (of the 256-value block at b, or the 32-value block for Q4_0) - reference kernels/q8.h:46-130 */
static void codes(uint32_t type, const uint8_t *b, int j, Codes *c)
{
  memset(c, 0, sizeof *c);
  switch (type)
  {
  case ORC_IQ2_XXS: /* q8.h:46-55 */
  {
    const uint8_t *q = b + 2 + 8 * j;
    const uint32_t aux = orc_ld32(q + 4);
    for (int k = 0; k < 4; k++)
      signed8(orc_grid_iq2xxs[q[k]], orc_ksigns[(aux >> (7 * k)) & 0x7F], c->w + 8 * k);
    c->s21[0] = c->s21[1] = 2 * (int)(aux >> 28) + 1;
    c->d = orc_f16(orc_ld16(b));
    break;
  }
  case ORC_IQ2_XS: /* q8.h:57-66 */
  {
    for (int k = 0; k < 4; k++)
    {
      const uint32_t q = orc_ld16(b + 2 + 2 * (4 * j + k));
      signed8(orc_grid_iq2xs[q & 511], orc_ksigns[q >> 9], c->w + 8 * k);
    }
    const uint32_t s = b[66 + j];
    c->s21[0] = 2 * (int)(s & 0x0F) + 1, c->s21[1] = 2 * (int)(s >> 4) + 1;
    c->d = orc_f16(orc_ld16(b));
    break;
  }
  case ORC_IQ1_M: /* q8.h:68-84 */
  {
    const uint64_t sc = orc_ld64(b + 48);
    const uint32_t s0 = (uint32_t)sc & 0xFFFF, s1 = (uint32_t)(sc >> 16) & 0xFFFF;
    const uint32_t s2 = (uint32_t)(sc >> 32) & 0xFFFF, s3 = (uint32_t)(sc >> 48);
    for (int k = 0; k < 4; k++)
    {
      const int kk = 4 * j + k;
      const uint32_t h = (b[32 + kk / 2] >> (4 * (kk % 2))) & 0x0F;
      iq1(orc_grid_iq1s[b[kk] | (h & 0x07) << 8], c->w + 8 * k);
      c->delta[k] = h & 0x08 ? -1 : 1;
    }
    for (int h = 0; h < 2; h++)
    {
      const int kk = 4 * j + 2 * h;
      c->s21[h] = 2 * (int)((sc >> (16 * (kk / 8) + 3 * ((kk / 2) % 4))) & 0x07) + 1;
    }
    c->d = orc_f16((s0 >> 12) | ((s1 >> 8) & 0x00F0) | ((s2 >> 4) & 0x0F00) | (s3 & 0xF000));
    break;
  }
  case ORC_IQ2_S: /* q8.h:86-95 */
  {
    for (int k = 0; k < 4; k++)
    {
      const int kk = 4 * j + k;
      signed8(orc_grid_iq2s[b[2 + kk] | ((b[66 + j] >> (2 * k)) & 0x03) << 8], b[34 + kk], c->w + 8 * k);
    }
    const uint32_t s = b[74 + j];
    c->s21[0] = 2 * (int)(s & 0x0F) + 1, c->s21[1] = 2 * (int)(s >> 4) + 1;
    c->d = orc_f16(orc_ld16(b));
    break;
  }
  case ORC_IQ3_XXS: /* q8.h:97-108 */
  {
    const uint8_t *q = b + 2 + 8 * j;
    const uint32_t aux = orc_ld32(b + 2 + 64 + 4 * j);
    for (int k = 0; k < 4; k++)
    {
      const uint64_t g = (uint64_t)orc_grid_iq3xxs[q[2 * k]] | (uint64_t)orc_grid_iq3xxs[q[2 * k + 1]] << 32;
      signed8(g, orc_ksigns[(aux >> (7 * k)) & 0x7F], c->w + 8 * k);
    }
    c->s21[0] = c->s21[1] = 2 * (2 * (int)(aux >> 28) + 1);
    c->d = orc_f16(orc_ld16(b));
    break;
  }
  case ORC_Q2_K: /* q8.h:110-118 */
  {
    const uint8_t *qs = b + 16 + 32 * (j / 4);
    const int shift = 2 * (j % 4);
    for (int i = 0; i < 32; i++)
      c->w[i] = (qs[i] >> shift) & 3;
    for (int h = 0; h < 2; h++)
      c->s21[h] = 8 * (b[2 * j + h] & 0x0F), c->m8[h] = 8 * (b[2 * j + h] >> 4);
    c->d = orc_f16(orc_ld16(b + 80)), c->dmin = orc_f16(orc_ld16(b + 82));
    c->has_min = 1;
    break;
  }
  case ORC_IQ1_S: /* q8.h:120-130 */
  {
    const uint32_t h = orc_ld16(b + 34 + 2 * j);
    for (int k = 0; k < 4; k++)
    {
      iq1(orc_grid_iq1s[b[2 + 4 * j + k] | ((h >> (3 * k)) & 0x07) << 8], c->w + 8 * k);
      c->delta[k] = h & 0x8000 ? -1 : 1;
    }
    c->s21[0] = c->s21[1] = 2 * (int)((h >> 12) & 0x07) + 1;
    c->d = orc_f16(orc_ld16(b));
    break;
  }
  case ORC_Q4_0: /* build-defined: ggml's Q4_0 codes (reference kernels/quant.h:240-248), one part, s21 8 */
  {
    for (int i = 0; i < 16; i++)
      c->w[i] = (b[2 + i] & 0x0F) - 8, c->w[16 + i] = (b[2 + i] >> 4) - 8;
    c->s21[0] = c->s21[1] = 8;
    c->d = orc_f16(orc_ld16(b));
    c->whole = 1;
    break;
  }
  case ORC_Q4_K: /* build-defined: group j of Q4_K (reference kernels/quant.h:89-103), one part with its minimum */
  {
    const uint8_t *s = b + 4;
    const int sc = j < 4 ? s[j] & 0x3F : (s[j + 4] & 0x0F) | ((s[j - 4] >> 2) & 0x30);
    const int m = j < 4 ? s[j + 4] & 0x3F : (s[j + 4] >> 4) | ((s[j] >> 2) & 0x30);
    const uint8_t *qs = b + 16 + (j / 2) * 32;
    for (int i = 0; i < 32; i++)
      c->w[i] = (qs[i] >> (4 * (j % 2))) & 0x0F;
    c->s21[0] = c->s21[1] = 8 * sc, c->m8[0] = c->m8[1] = 8 * m;
    c->d = orc_f16(orc_ld16(b)), c->dmin = orc_f16(orc_ld16(b + 2));
    c->has_min = 1, c->whole = 1;
    break;
  }
  case ORC_Q3_K: /* build-defined: values 32j .. 32j + 31 of Q3_K (reference kernels/quant.h:264-284), two halves */
  {
    const uint8_t *sc = b + 96;
    for (int i = 0; i < 32; i++)
    {
      const int v = 32 * j + i, n = v / 128, r = v % 128, jj = r / 32;
      const int q2 = (b[32 + 32 * n + r % 32] >> (2 * jj)) & 3;
      const int hb = (b[r % 32] >> (4 * n + jj)) & 1;
      c->w[i] = q2 - (hb ? 0 : 4);
    }
    for (int h = 0; h < 2; h++)
    {
      const int g = 2 * j + h, grp = g / 4, w = g % 4;
      const int low = ((grp & 1 ? sc[4 + w] : sc[w]) >> (grp & 2 ? 4 : 0)) & 0x0F;
      const int sc6 = low | ((sc[8 + w] >> (2 * grp)) & 0x03) << 4;
      c->s21[h] = 8 * (sc6 - 32);
    }
    c->d = orc_f16(orc_ld16(b + 108));
    break;
  }
  default: abort();
  }
}

/* the block's sum before x's scale: reference kernels/q8.h:133-162 (halves), src/cpu/q8.c:282-312 */
static float block_sub(uint32_t type, const Codes *c, const int8_t *x)
{
  int isum[2] = {0, 0}, xsum[2] = {0, 0};
  for (int h = 0; h < 2; h++)
    for (int k = 2 * h; k < 2 * h + 2; k++)
    {
      int gx = 0, sx = 0;
      for (int i = 0; i < 8; i++)
        gx += c->w[8 * k + i] * x[8 * k + i], sx += x[8 * k + i];
      if (type == ORC_IQ1_M || type == ORC_IQ1_S)
        isum[h] += 8 * gx + c->delta[k] * sx;
      else
        isum[h] += gx;
      xsum[h] += sx;
    }
  if (c->whole)
  {
    const int is = isum[0] + isum[1], xs = xsum[0] + xsum[1];
    return c->has_min ? part(c->d, c->s21[0], is) - part(c->dmin, c->m8[0], xs) : part(c->d, c->s21[0], is);
  }
  if (c->has_min)
    return (part(c->d, c->s21[0], isum[0]) - part(c->dmin, c->m8[0], xsum[0])) +
           (part(c->d, c->s21[1], isum[1]) - part(c->dmin, c->m8[1], xsum[1]));
  return part(c->d, c->s21[0], isum[0]) + part(c->d, c->s21[1], isum[1]);
}

float orc_lane_sub(uint32_t type, const uint8_t *row, uint32_t s, const int8_t *xb)
{
  orc_init();
  const uint32_t per = orc_block_values(type) / LANE_VALUES;
  Codes c;
  codes(type, row + (s / per) * orc_block_bytes(type), (int)(s % per), &c);
  return block_sub(type, &c, xb);
}

/* reference kernels/q8.h:263-277, src/cpu/q8.c:409-427, kernels/lane.h:54-56 */
bool orc_q8_round(const float *x, uint32_t rows, uint32_t cols, uint32_t xs, int8_t *q, float *d)
{
  if (!x || !q || !d || !rows || !cols || cols % LANE_VALUES || xs < cols)
    return false;
  const uint32_t nb = cols / LANE_VALUES;
  for (uint32_t r = 0; r < rows; r++)
    for (uint32_t s = 0; s < nb; s++)
    {
      const float *xb = x + (uint64_t)r * xs + (uint64_t)s * LANE_VALUES;
      float a = 0.0f;
      for (int i = 0; i < LANE_VALUES; i++)
        a = fmaxf(a, fabsf(xb[i]));
      const float inv = a > 0.0f ? 127.0f / a : 0.0f;
      for (int i = 0; i < LANE_VALUES; i++)
        q[(uint64_t)r * cols + (uint64_t)s * LANE_VALUES + i] = (int8_t)(int)rintf(xb[i] * inv);
      d[(uint64_t)r * nb + s] = a / 127.0f;
    }
  return true;
}

/* one row, one token: the lane assignment and the tree (reference kernels/q8.h:197-210, tests/test_cpu_q8.c:139-162) */
static float row_sum(uint32_t type, const uint8_t *row, uint32_t cols, const int8_t *q, const float *qd)
{
  const uint32_t L = LANE_LANES(cols), per = orc_block_values(type) / LANE_VALUES, bb = orc_block_bytes(type);
  float acc[32] = {0}, nx[32];
  for (uint32_t s = 0; s < cols / LANE_VALUES; s++)
  {
    Codes c;
    codes(type, row + (s / per) * bb, (int)(s % per), &c);
    acc[s % L] = fmaf(qd[s], block_sub(type, &c, q + (uint64_t)s * LANE_VALUES), acc[s % L]);
  }
  for (uint32_t o = L / 2; o > 0; o >>= 1)
  {
    for (uint32_t l = 0; l < L; l++)
      nx[l] = acc[l] + acc[l ^ o];
    memcpy(acc, nx, sizeof nx);
  }
  return acc[0];
}

/* reference src/cpu/q8.c:383-407 (its semantics: tokens at q + t cols, their scales at d + t cols / 32, y at
   y + t ys + r) */
bool orc_q8_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t *q, const float *d,
                 uint32_t n, float *y, uint32_t ys)
{
  orc_init();
  const uint32_t bv = orc_block_values(type);
  if (!orc_lane_known(type) || !w || !q || !d || !y || !n || !cols || cols % bv || cols % LANE_VALUES || r1 < r0)
    return false;
  const uint32_t nb = cols / LANE_VALUES;
  const uint64_t row_bytes = (uint64_t)(cols / bv) * orc_block_bytes(type);
  for (uint32_t t = 0; t < n; t++)
    for (uint32_t r = r0; r < r1; r++)
      y[(uint64_t)t * ys + r] = row_sum(type, (const uint8_t *)w + r * row_bytes, cols, q + (uint64_t)t * cols,
                                        d + (uint64_t)t * nb);
  return true;
}
