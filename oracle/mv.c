/* TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h): the fp32 matvec contract, scalar.

   reference: kernels/quant.h:60-348 (each type's exact dequantisation, 8 values a chunk, every product rounded on its
   own), kernels/mv.h:12-70 (a row's order: lane l of 32 sums its chunks l, l + 32, ... in order, 8 fmaf a chunk, then
   the xor tree o = 16 .. 1), src/cpu/expert.c:140-253 (the CPU twin of the same order). built with -ffp-contract=off. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "orc_internal.h"

#define CHUNK 8
#define LANES 32
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

bool orc_mv_known(uint32_t type)
{
  switch (type)
  {
  case ORC_F32:
  case ORC_BF16:
  case ORC_Q4_0:
  case ORC_Q8_0:
  case ORC_IQ4_NL:
  case ORC_Q2_K:
  case ORC_Q3_K:
  case ORC_Q4_K:
  case ORC_Q5_K:
  case ORC_Q6_K:
  case ORC_IQ2_XXS:
  case ORC_IQ2_XS:
  case ORC_IQ3_XXS:
  case ORC_IQ1_S:
  case ORC_IQ2_S:
  case ORC_IQ4_XS:
  case ORC_IQ1_M: return true;
  default: return false;
  }
}

static void sgn8(float db, uint64_t grid, uint32_t signs, float *v)
{
  for (int j = 0; j < CHUNK; j++)
  {
    const float x = db * (float)(uint8_t)(grid >> (8 * j));
    v[j] = (signs >> j) & 1 ? -x : x;
  }
}

static void k_scale_min(const uint8_t *s, int g, int *sc, int *m)
{
  *sc = g < 4 ? s[g] & 0x3F : (s[g + 4] & 0x0F) | ((s[g - 4] >> 2) & 0x30);
  *m = g < 4 ? s[g + 4] & 0x3F : (s[g + 4] >> 4) | ((s[g] >> 2) & 0x30);
}

/* chunk k (values 8k .. 8k + 7) of the block at b: reference kernels/quant.h decode<T> */
static void decode(uint32_t type, const uint8_t *b, int k, float *v)
{
  switch (type)
  {
  case ORC_F32: memcpy(v, b, 32); break; /* a chunk of 8 floats */
  case ORC_BF16:
    for (int j = 0; j < CHUNK; j++)
    {
      const uint32_t u = orc_ld16(b + 2 * j) << 16;
      memcpy(&v[j], &u, 4);
    }
    break;
  case ORC_Q8_0: /* quant.h:66-69 */
  {
    const float d = orc_f16(orc_ld16(b));
    for (int j = 0; j < CHUNK; j++)
      v[j] = (float)(int8_t)b[2 + k * CHUNK + j] * d;
    break;
  }
  case ORC_Q4_0: /* quant.h:242-248 */
  {
    const float d = orc_f16(orc_ld16(b));
    const uint8_t *qs = b + 2 + (k % 2) * CHUNK;
    for (int j = 0; j < CHUNK; j++)
      v[j] = d * (float)((int)((qs[j] >> (4 * (k / 2))) & 0x0F) - 8);
    break;
  }
  case ORC_IQ4_NL: /* quant.h:199-205 */
  {
    const float d = orc_f16(orc_ld16(b));
    const uint8_t *qs = b + 2 + (k % 2) * CHUNK;
    for (int j = 0; j < CHUNK; j++)
      v[j] = d * (float)kIq4nl[(qs[j] >> (4 * (k / 2))) & 0x0F];
    break;
  }
  case ORC_Q4_K: /* quant.h:91-103: (d * sc) * q - (dmin * m), the subtract rounded once */
  {
    const int g = k / 4, l0 = (k % 4) * CHUNK;
    int sc, m;
    k_scale_min(b + 4, g, &sc, &m);
    const float d = orc_f16(orc_ld16(b)) * (float)sc, dm = orc_f16(orc_ld16(b + 2)) * (float)m;
    const uint8_t *qs = b + 16 + (g / 2) * 32 + l0;
    for (int j = 0; j < CHUNK; j++)
      v[j] = d * (float)((qs[j] >> (4 * (g % 2))) & 0x0F) - dm;
    break;
  }
  case ORC_Q5_K: /* quant.h:73-87 */
  {
    const int g = k / 4, l0 = (k % 4) * CHUNK;
    int sc, m;
    k_scale_min(b + 4, g, &sc, &m);
    const float d = orc_f16(orc_ld16(b)) * (float)sc, dm = orc_f16(orc_ld16(b + 2)) * (float)m;
    const uint8_t *qh = b + 16 + l0, *qs = b + 48 + (g / 2) * 32 + l0;
    for (int j = 0; j < CHUNK; j++)
    {
      const int q = ((qs[j] >> (4 * (g % 2))) & 0x0F) | (((qh[j] >> g) & 1) << 4);
      v[j] = d * (float)q - dm;
    }
    break;
  }
  case ORC_Q6_K: /* quant.h:166-179 */
  {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d0 = orc_f16(orc_ld16(b + 208));
    const int g = k / 4, h = g / 4, r = g % 4, l0 = (k % 4) * CHUNK;
    const float d = d0 * (float)sc[(g * 32 + l0) / 16];
    for (int j = 0; j < CHUNK; j++)
    {
      const int l = l0 + j;
      const int lo = (ql[h * 64 + (r % 2) * 32 + l] >> (4 * (r / 2))) & 0x0F;
      const int hi = (qh[h * 32 + l] >> (2 * r)) & 0x03;
      v[j] = d * (float)((lo | hi << 4) - 32);
    }
    break;
  }
  case ORC_Q2_K: /* quant.h:254-262 */
  {
    const int g = k / 2, l0 = (k % 4) * CHUNK, shift = 2 * ((k % 16) / 4);
    const uint8_t *qs = b + 16 + 32 * (k / 16) + l0;
    const float dl = orc_f16(orc_ld16(b + 80)) * (float)(b[g] & 0x0F);
    const float ml = orc_f16(orc_ld16(b + 82)) * (float)(b[g] >> 4);
    for (int j = 0; j < CHUNK; j++)
      v[j] = dl * (float)((qs[j] >> shift) & 0x03) - ml;
    break;
  }
  case ORC_Q3_K: /* quant.h:264-284 */
  {
    const int i0 = k * CHUNK, n = i0 / 128, r = i0 % 128, j = r / 32, sub = (r % 32) / 16, l0 = r % 16;
    const int g = 8 * n + 2 * j + sub, grp = g / 4, w = g % 4;
    const uint8_t *sc = b + 96;
    const int low = ((grp & 1 ? sc[4 + w] : sc[w]) >> (grp & 2 ? 4 : 0)) & 0x0F;
    const int sc6 = low | ((sc[8 + w] >> (2 * grp)) & 0x03) << 4;
    const float dl = orc_f16(orc_ld16(b + 108)) * (float)(sc6 - 32);
    const uint8_t *qs = b + 32 + 32 * n + 16 * sub + l0, *hm = b + 16 * sub + l0;
    const int bit = 4 * n + j;
    for (int jj = 0; jj < CHUNK; jj++)
      v[jj] = dl * (float)(((qs[jj] >> (2 * j)) & 0x03) - ((hm[jj] >> bit) & 1 ? 0 : 4));
    break;
  }
  case ORC_IQ2_XXS: /* quant.h:183-197: ((d * (0.5 + s)) * 0.25) * grid, signed */
  {
    const uint8_t *q = b + 2 + (k / 4) * 8;
    const uint32_t aux = orc_ld32(q + 4);
    const float db = orc_f16(orc_ld16(b)) * (0.5f + (float)(aux >> 28)) * 0.25f;
    sgn8(db, orc_grid_iq2xxs[q[k % 4]], orc_ksigns[(aux >> (7 * (k % 4))) & 0x7F], v);
    break;
  }
  case ORC_IQ2_XS: /* quant.h:199-210 */
  {
    const uint32_t q = orc_ld16(b + 2 + 2 * k);
    const int s = (b[66 + k / 4] >> (4 * ((k / 2) % 2))) & 0x0F;
    const float db = orc_f16(orc_ld16(b)) * (0.5f + (float)s) * 0.25f;
    sgn8(db, orc_grid_iq2xs[q & 511], orc_ksigns[q >> 9], v);
    break;
  }
  case ORC_IQ2_S: /* quant.h:300-311 */
  {
    const int s = (b[74 + k / 4] >> (4 * ((k / 2) % 2))) & 0x0F;
    const float db = orc_f16(orc_ld16(b)) * (0.5f + (float)s) * 0.25f;
    sgn8(db, orc_grid_iq2s[b[2 + k] | ((b[66 + k / 4] >> (2 * (k % 4))) & 0x03) << 8], b[34 + k], v);
    break;
  }
  case ORC_IQ3_XXS: /* quant.h:219-230: ((d * (0.5 + s)) * 0.5) * grid, signed */
  {
    const uint8_t *q = b + 2 + (k / 4) * 8 + (k % 4) * 2;
    const uint32_t aux = orc_ld32(b + 2 + 64 + (k / 4) * 4);
    const float db = orc_f16(orc_ld16(b)) * (0.5f + (float)(aux >> 28)) * 0.5f;
    const uint64_t grid = (uint64_t)orc_grid_iq3xxs[q[0]] | (uint64_t)orc_grid_iq3xxs[q[1]] << 32;
    sgn8(db, grid, orc_ksigns[(aux >> (7 * (k % 4))) & 0x7F], v);
    break;
  }
  case ORC_IQ4_XS: /* quant.h:232-240 */
  {
    const int g = k / 4, j0 = (k % 4) * CHUNK;
    const int ls = ((b[4 + g / 2] >> (4 * (g % 2))) & 0x0F) | ((orc_ld16(b + 2) >> (2 * g)) & 0x03) << 4;
    const float dl = orc_f16(orc_ld16(b)) * (float)(ls - 32);
    const uint8_t *qs = b + 8 + 16 * g + j0 % 16;
    for (int j = 0; j < CHUNK; j++)
      v[j] = dl * (float)kIq4nl[(qs[j] >> (4 * (j0 / 16))) & 0x0F];
    break;
  }
  case ORC_IQ1_S: /* quant.h:315-321: (d * (2s + 1)) * (grid + delta) */
  {
    const uint32_t h = orc_ld16(b + 34 + 2 * (k / 4));
    const float dl = orc_f16(orc_ld16(b)) * (float)(2 * ((h >> 12) & 0x07) + 1);
    const float delta = h & 0x8000 ? -0.125f : 0.125f;
    const uint64_t grid = orc_grid_iq1s[b[2 + k] | ((h >> (3 * (k % 4))) & 0x07) << 8];
    for (int j = 0; j < CHUNK; j++)
      v[j] = dl * ((float)(int8_t)(uint8_t)(grid >> (8 * j)) + delta);
    break;
  }
  case ORC_IQ1_M: /* quant.h:322-336 */
  {
    const uint8_t *qs = b, *qh = b + 32;
    const uint64_t sc = orc_ld64(b + 48);
    const uint32_t s0 = (uint32_t)sc & 0xFFFF, s1 = (uint32_t)(sc >> 16) & 0xFFFF;
    const uint32_t s2 = (uint32_t)(sc >> 32) & 0xFFFF, s3 = (uint32_t)(sc >> 48);
    const float d = orc_f16((s0 >> 12) | ((s1 >> 8) & 0x00F0) | ((s2 >> 4) & 0x0F00) | (s3 & 0xF000));
    const int s = (int)((sc >> (16 * (k / 8) + 3 * ((k / 2) % 4))) & 0x07);
    const float dl = d * (float)(2 * s + 1);
    const uint32_t h = (qh[k / 2] >> (4 * (k % 2))) & 0x0F;
    const float delta = h & 0x08 ? -0.125f : 0.125f;
    const uint64_t grid = orc_grid_iq1s[qs[k] | (h & 0x07) << 8];
    for (int j = 0; j < CHUNK; j++)
      v[j] = dl * ((float)(int8_t)(uint8_t)(grid >> (8 * j)) + delta);
    break;
  }
  default: abort();
  }
}

/* where chunk c of a row lies: block c / per, chunk c % per of it (reference kernels/quant.h:124-135) */
static const uint8_t *chunk_at(uint32_t type, const uint8_t *row, uint32_t c, int *k)
{
  const uint32_t bv = orc_block_values(type);
  if (bv == 1)
  { /* F32 / BF16: a chunk is 8 values */
    *k = 0;
    return row + (uint64_t)c * CHUNK * orc_block_bytes(type);
  }
  const uint32_t per = bv / CHUNK;
  *k = (int)(c % per);
  return row + (uint64_t)(c / per) * orc_block_bytes(type);
}

bool orc_dequant(uint32_t type, const void *src, uint64_t values, float *dst)
{
  orc_init();
  const uint32_t bv = orc_block_values(type);
  if (!orc_mv_known(type) || values % CHUNK || values % bv)
    return false;
  for (uint64_t c = 0; c < values / CHUNK; c++)
  {
    int k;
    const uint8_t *b = chunk_at(type, (const uint8_t *)src, (uint32_t)c, &k);
    decode(type, b, k, dst + c * CHUNK);
  }
  return true;
}

static uint64_t row_bytes(uint32_t type, uint32_t cols)
{
  return (uint64_t)(cols / orc_block_values(type)) * orc_block_bytes(type);
}

/* reference kernels/mv.h:45-70 (rows_of) */
bool orc_mv_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const float *x, uint32_t xs,
                 uint32_t n, float *y, uint32_t ys)
{
  orc_init();
  if (!orc_mv_known(type) || !w || !x || !y || !cols || cols % orc_block_values(type) || cols % CHUNK || r1 < r0)
    return false;
  const uint32_t chunks = cols / CHUNK;
  for (uint32_t r = r0; r < r1; r++)
  {
    const uint8_t *row = (const uint8_t *)w + (uint64_t)r * row_bytes(type, cols);
    for (uint32_t t = 0; t < n; t++)
    {
      const float *xt = x + (uint64_t)t * xs;
      float acc[LANES] = {0}, nx[LANES];
      for (uint32_t c = 0; c < chunks; c++)
      {
        float v[CHUNK];
        int k = 0;
        const uint8_t *b = chunk_at(type, row, c, &k);
        decode(type, b, k, v);
        float s = acc[c % LANES];
        for (int j = 0; j < CHUNK; j++)
          s = fmaf(v[j], xt[(uint64_t)c * CHUNK + j], s);
        acc[c % LANES] = s;
      }
      for (uint32_t o = LANES / 2; o > 0; o >>= 1)
      {
        for (uint32_t l = 0; l < LANES; l++)
          nx[l] = acc[l] + acc[l ^ o];
        memcpy(acc, nx, sizeof nx);
      }
      y[(uint64_t)t * ys + r] = acc[0];
    }
  }
  return true;
}
